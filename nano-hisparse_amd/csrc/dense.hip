// Elementwise stages of the batched decode layer, fused: residual add +
// RMSNorm, rotary embedding of q and k in place, and SiLU(gate) * up. Each
// reproduces the rounding steps of the torch expression it replaces (every
// torch bf16/fp16 operation computes in fp32 and rounds its result to the
// tensor dtype; separate torch operations never fuse a multiply into an
// add, hence fp contract(off)), so only reduction order can differ.
#include "nhs_common.h"

namespace nhs {

constexpr int kNormThreads = 512;
constexpr int kNormHeld = 32;  // elements per thread held in registers (rows up to 16384)

template <typename T>
__device__ __forceinline__ float rnd(float v) {
  return T::to_float(T::from_float(v));
}

struct F32T {
  using Bits = float;
  __device__ static float to_float(float b) { return b; }
  __device__ static float from_float(float v) { return v; }
};
struct BF16T {
  using Bits = uint16_t;
  __device__ static float to_float(uint16_t b) { return bf16_bits_to_f32(b); }
  __device__ static uint16_t from_float(float v) { return f32_to_bf16_bits(v); }
};
struct F16T {
  using Bits = uint16_t;
  __device__ static float to_float(uint16_t b) { return f16_bits_to_f32(b); }
  __device__ static uint16_t from_float(float v) { return f32_to_f16_bits(v); }
};

// h = x + delta (rounded; delta may be null), written back to x when
// write_back; out = round(round(h * rsqrt(mean(h^2) + eps)) * weight).
// One workgroup per row.
template <typename T>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(typename T::Bits* x, const typename T::Bits* delta,
                                                                   const typename T::Bits* weight,
                                                                   typename T::Bits* out, int width, float eps,
                                                                   int write_back) {
#pragma clang fp contract(off)
  __shared__ float partial[kNormThreads / kWave];
  const int row = blockIdx.x;
  typename T::Bits* xr = x + (int64_t)row * width;
  const typename T::Bits* dr = delta ? delta + (int64_t)row * width : nullptr;
  // rows of up to kNormThreads * kNormHeld elements are held in registers:
  // every load is issued before the first store, which could alias them
  float held[kNormHeld], wv[kNormHeld];
  float acc = 0.f;
  const bool in_regs = width <= kNormThreads * kNormHeld;
  if (in_regs) {
    // x, delta and the weights are all requested before the first use
#pragma unroll
    for (int j = 0; j < kNormHeld; ++j) {
      const int i = threadIdx.x + j * kNormThreads;
      held[j] = i < width ? T::to_float(xr[i]) : 0.f;
      wv[j] = i < width ? T::to_float(weight[i]) : 0.f;
    }
    if (dr) {
      float dv[kNormHeld];
#pragma unroll
      for (int j = 0; j < kNormHeld; ++j) {
        const int i = threadIdx.x + j * kNormThreads;
        dv[j] = i < width ? T::to_float(dr[i]) : 0.f;
      }
#pragma unroll
      for (int j = 0; j < kNormHeld; ++j) held[j] = rnd<T>(held[j] + dv[j]);
      if (write_back)
#pragma unroll
        for (int j = 0; j < kNormHeld; ++j) {
          const int i = threadIdx.x + j * kNormThreads;
          if (i < width) xr[i] = T::from_float(held[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < kNormHeld; ++j) acc += held[j] * held[j];
  } else {
    for (int i = threadIdx.x; i < width; i += kNormThreads) {
      float h = T::to_float(xr[i]);
      if (dr) {
        h = rnd<T>(h + T::to_float(dr[i]));
        if (write_back) xr[i] = T::from_float(h);
      }
      acc += h * h;
    }
  }
  acc = group_sum(acc, kWave);
  if ((threadIdx.x & (kWave - 1)) == 0) partial[threadIdx.x / kWave] = acc;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / kWave; ++w) total += partial[w];
  const float r = rsqrtf(total / (float)width + eps);
  typename T::Bits* orow = out + (int64_t)row * width;
  if (in_regs) {
#pragma unroll
    for (int j = 0; j < kNormHeld; ++j) {
      const int i = threadIdx.x + j * kNormThreads;
      if (i < width) orow[i] = T::from_float(rnd<T>(held[j] * r) * wv[j]);
    }
  } else {
    for (int i = threadIdx.x; i < width; i += kNormThreads) {
      float h = T::to_float(xr[i]);
      if (dr && !write_back) h = rnd<T>(h + T::to_float(dr[i]));
      orow[i] = T::from_float(rnd<T>(h * r) * T::to_float(weight[i]));
    }
  }
}

// add_rmsnorm for 16-bit rows of a multiple of 8 elements, at most
// V * kNormThreads * 8: thread t owns the 8-element chunks t,
// t + kNormThreads, ... below width / 8 and moves them with 16-byte loads
// and stores. Same arithmetic as add_rmsnorm_kernel.
template <typename T, int V>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_vec_kernel(uint16_t* x, const uint16_t* delta,
                                                                       const uint16_t* weight, uint16_t* out,
                                                                       int width, float eps, int write_back) {
#pragma clang fp contract(off)
  __shared__ float partial[kNormThreads / kWave];
  const int row = blockIdx.x;
  uint4* xr = reinterpret_cast<uint4*>(x + (int64_t)row * width);
  const uint4* dr = delta ? reinterpret_cast<const uint4*>(delta + (int64_t)row * width) : nullptr;
  const uint4* wr = reinterpret_cast<const uint4*>(weight);
  const int chunks = width >> 3;
  uint4 xv[V], dv[V], wv[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    // a chunk past the row reads as zeros and adds nothing to the sum
    const int c = threadIdx.x + j * kNormThreads;
    const bool ok = c < chunks;
    xv[j] = ok ? xr[c] : make_uint4(0u, 0u, 0u, 0u);
    wv[j] = ok ? wr[c] : make_uint4(0u, 0u, 0u, 0u);
    dv[j] = dr && ok ? dr[c] : make_uint4(0u, 0u, 0u, 0u);
  }
  float h[V][8];
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const uint32_t xw[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
    const uint32_t dw[4] = {dv[j].x, dv[j].y, dv[j].z, dv[j].w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = T::to_float((uint16_t)(xw[e >> 1] >> ((e & 1) * 16)));
      if (dr) v = rnd<T>(v + T::to_float((uint16_t)(dw[e >> 1] >> ((e & 1) * 16))));
      h[j][e] = v;
      acc += v * v;
      const uint32_t bits = T::from_float(v);
      o[e >> 1] = (e & 1) ? (o[e >> 1] | (bits << 16)) : bits;
    }
    if (dr && write_back && threadIdx.x + j * kNormThreads < chunks)
      xr[threadIdx.x + j * kNormThreads] = make_uint4(o[0], o[1], o[2], o[3]);
  }
  acc = group_sum(acc, kWave);
  if ((threadIdx.x & (kWave - 1)) == 0) partial[threadIdx.x / kWave] = acc;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / kWave; ++w) total += partial[w];
  const float r = rsqrtf(total / (float)width + eps);
  uint4* orow = reinterpret_cast<uint4*>(out + (int64_t)row * width);
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const uint32_t ww[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float w = T::to_float((uint16_t)(ww[e >> 1] >> ((e & 1) * 16)));
      const uint32_t bits = T::from_float(rnd<T>(h[j][e] * r) * w);
      o[e >> 1] = (e & 1) ? (o[e >> 1] | (bits << 16)) : bits;
    }
    if (threadIdx.x + j * kNormThreads < chunks) orow[threadIdx.x + j * kNormThreads] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Rotary embedding in place on rows of [heads, head_dim] (q heads then kv
// heads of one fused projection row): for d < D/2 with lo = t[d],
// hi = t[d + D/2], c = cos[row, d], s = sin[row, d]:
//   t[d]       = round(round(lo * c) + round(-hi * s))
//   t[d + D/2] = round(round(hi * c) + round(lo * s))
// One thread per (row, head, d).
template <typename T>
__global__ void rope_kernel(typename T::Bits* t, int64_t row_stride, int heads, int half,
                            const typename T::Bits* cos, const typename T::Bits* sin, int64_t total) {
#pragma clang fp contract(off)
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int per_row = heads * half;
  const int row = (int)(idx / per_row);
  const int rem = (int)(idx - (int64_t)row * per_row);
  const int head = rem / half, d = rem - head * half;
  typename T::Bits* p = t + (int64_t)row * row_stride + (int64_t)head * 2 * half;
  const float lo = T::to_float(p[d]), hi = T::to_float(p[d + half]);
  const float c = T::to_float(cos[(int64_t)row * half + d]), s = T::to_float(sin[(int64_t)row * half + d]);
  p[d] = T::from_float(rnd<T>(lo * c) + rnd<T>(-hi * s));
  p[d + half] = T::from_float(rnd<T>(hi * c) + rnd<T>(lo * s));
}

// out[row, i] = round(round(silu(g)) * u), g = gu[row, i], u = gu[row, inter + i].
template <typename T>
__global__ void silu_mul_kernel(const typename T::Bits* gu, typename T::Bits* out, int inter, int64_t total) {
#pragma clang fp contract(off)
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int64_t row = idx / inter;
  const int i = (int)(idx - row * inter);
  const float g = T::to_float(gu[row * 2 * inter + i]);
  const float u = T::to_float(gu[row * 2 * inter + inter + i]);
  const float s = rnd<T>(g / (1.0f + expf(-g)));
  out[idx] = T::from_float(s * u);
}

}  // namespace nhs

using namespace nhs;

extern "C" int nhs_add_rmsnorm(int32_t rows, int32_t width, int32_t dtype, void* x, const void* delta,
                               int32_t write_back, const void* weight, float eps, void* out, void* stream) {
  const LaunchEvents ev = take_launch_events();
  if (!x || !weight || !out) return fail(NHS_ERR_INVALID, "nhs_add_rmsnorm: null pointer");
  if (rows < 0 || width < 1 || !valid_dtype(dtype)) return fail(NHS_ERR_INVALID, "nhs_add_rmsnorm: bad shape/dtype");
  if (rows == 0) return NHS_OK;
  const int wb = delta && write_back ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)rows), block(kNormThreads);
  const int per_pass = kNormThreads * 8;  // elements of one chunk per thread
  const bool aligned = (((uintptr_t)x | (uintptr_t)delta | (uintptr_t)weight | (uintptr_t)out) % 16) == 0;
  if (dtype != NHS_F32 && aligned && width % 8 == 0 && (width + per_pass - 1) / per_pass <= 4) {
    const int v = (width + per_pass - 1) / per_pass;
    auto* xp = static_cast<uint16_t*>(x);
    auto* dp = static_cast<const uint16_t*>(delta);
    auto* wp = static_cast<const uint16_t*>(weight);
    auto* op = static_cast<uint16_t*>(out);
#define NHS_NORM_VEC(TT, VV) \
  launch(add_rmsnorm_vec_kernel<TT, VV>, grid, block, 0, s, ev.start, ev.stop, xp, dp, wp, op, width, eps, wb)
    if (dtype == NHS_BF16) {
      if (v == 1) NHS_NORM_VEC(BF16T, 1); else if (v == 2) NHS_NORM_VEC(BF16T, 2);
      else if (v == 3) NHS_NORM_VEC(BF16T, 3); else NHS_NORM_VEC(BF16T, 4);
    } else {
      if (v == 1) NHS_NORM_VEC(F16T, 1); else if (v == 2) NHS_NORM_VEC(F16T, 2);
      else if (v == 3) NHS_NORM_VEC(F16T, 3); else NHS_NORM_VEC(F16T, 4);
    }
#undef NHS_NORM_VEC
    return launch_status("nhs_add_rmsnorm");
  }
  if (dtype == NHS_BF16)
    launch(add_rmsnorm_kernel<BF16T>, grid, block, 0, s, ev.start, ev.stop, static_cast<uint16_t*>(x),
           static_cast<const uint16_t*>(delta), static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out),
           width, eps, wb);
  else if (dtype == NHS_F16)
    launch(add_rmsnorm_kernel<F16T>, grid, block, 0, s, ev.start, ev.stop, static_cast<uint16_t*>(x),
           static_cast<const uint16_t*>(delta), static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out),
           width, eps, wb);
  else
    launch(add_rmsnorm_kernel<F32T>, grid, block, 0, s, ev.start, ev.stop, static_cast<float*>(x),
           static_cast<const float*>(delta), static_cast<const float*>(weight), static_cast<float*>(out), width,
           eps, wb);
  return launch_status("nhs_add_rmsnorm");
}

extern "C" int nhs_rope(int32_t rows, int32_t heads, int32_t head_dim, int32_t dtype, void* t, int64_t row_stride,
                        const void* cos, const void* sin, void* stream) {
  const LaunchEvents ev = take_launch_events();
  if (!t || !cos || !sin) return fail(NHS_ERR_INVALID, "nhs_rope: null pointer");
  if (rows < 0 || heads < 1 || head_dim < 2 || head_dim % 2 || !valid_dtype(dtype) ||
      row_stride < (int64_t)heads * head_dim)
    return fail(NHS_ERR_INVALID, "nhs_rope: bad shape/dtype");
  if (rows == 0) return NHS_OK;
  const int half = head_dim / 2;
  const int64_t total = (int64_t)rows * heads * half;
  const int threads = 256;
  const dim3 grid((unsigned)((total + threads - 1) / threads)), block(threads);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == NHS_BF16)
    launch(rope_kernel<BF16T>, grid, block, 0, s, ev.start, ev.stop, static_cast<uint16_t*>(t), row_stride, heads,
           half, static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin), total);
  else if (dtype == NHS_F16)
    launch(rope_kernel<F16T>, grid, block, 0, s, ev.start, ev.stop, static_cast<uint16_t*>(t), row_stride, heads,
           half, static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin), total);
  else
    launch(rope_kernel<F32T>, grid, block, 0, s, ev.start, ev.stop, static_cast<float*>(t), row_stride, heads, half,
           static_cast<const float*>(cos), static_cast<const float*>(sin), total);
  return launch_status("nhs_rope");
}

extern "C" int nhs_silu_mul(int32_t rows, int32_t inter, int32_t dtype, const void* gate_up, void* out,
                            void* stream) {
  const LaunchEvents ev = take_launch_events();
  if (!gate_up || !out) return fail(NHS_ERR_INVALID, "nhs_silu_mul: null pointer");
  if (rows < 0 || inter < 1 || !valid_dtype(dtype)) return fail(NHS_ERR_INVALID, "nhs_silu_mul: bad shape/dtype");
  if (rows == 0) return NHS_OK;
  const int64_t total = (int64_t)rows * inter;
  const int threads = 256;
  const dim3 grid((unsigned)((total + threads - 1) / threads)), block(threads);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == NHS_BF16)
    launch(silu_mul_kernel<BF16T>, grid, block, 0, s, ev.start, ev.stop, static_cast<const uint16_t*>(gate_up),
           static_cast<uint16_t*>(out), inter, total);
  else if (dtype == NHS_F16)
    launch(silu_mul_kernel<F16T>, grid, block, 0, s, ev.start, ev.stop, static_cast<const uint16_t*>(gate_up),
           static_cast<uint16_t*>(out), inter, total);
  else
    launch(silu_mul_kernel<F32T>, grid, block, 0, s, ev.start, ev.stop, static_cast<const float*>(gate_up),
           static_cast<float*>(out), inter, total);
  return launch_status("nhs_silu_mul");
}
