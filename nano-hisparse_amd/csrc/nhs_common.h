// Shared device helpers for the gfx950 sparse-decode kernels: element
// conversion, wave64 cross-lane sums and block-wide scans.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nhs.h"

namespace nhs {

// Records a message for nhs_last_error() and returns `code`.
int fail(int code, const char* fmt, ...);
// Converts the launch status of the kernels just enqueued into an nhs status.
int launch_status(const char* what);

// Timing events set by nhs_set_launch_events for the next entry point called
// on this thread; take_launch_events() returns and clears them.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
LaunchEvents take_launch_events();

// Enqueues `kernel`. With a start and/or stop event the launch goes through
// hipExtLaunchKernel, which stamps the events with the dispatch's own begin
// and end times (no marker packets between them and the kernel).
template <typename K, typename... Args>
inline void launch(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream, hipEvent_t start,
                   hipEvent_t stop, Args... args) {
  if (start || stop)
    hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, stream, start, stop, 0u, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
}

constexpr int kWave = 64;

inline int elem_size(int dtype) { return dtype == NHS_F32 ? 4 : 2; }
inline bool valid_dtype(int dtype) { return dtype == NHS_F32 || dtype == NHS_F16 || dtype == NHS_BF16; }
inline int ilog2(int v) {
  int r = 0;
  while ((1 << r) < v) ++r;
  return r;
}

// Division of 32-bit unsigned values by a runtime-invariant divisor d >= 1
// without a hardware divide: q = (umulhi(n, magic) + n) >> shift, with
// shift = ceil(log2 d) and magic = floor(2^32 (2^shift - d) / d) + 1
// (the round-up method of Hacker's Delight, ch. 10; exact for all n < 2^32).
struct FastDiv {
  uint32_t d, magic, shift;
  FastDiv() = default;
  explicit FastDiv(uint32_t divisor) : d(divisor) {
    shift = 0;
    while ((1ull << shift) < divisor) ++shift;
    magic = (uint32_t)((((1ull << shift) - divisor) << 32) / divisor + 1);
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    uint64_t t = __umulhi(n, magic);
    return (uint32_t)((t + n) >> shift);
  }
};

// ---- element conversion -------------------------------------------------

// Pointers known to address global memory: loads and stores through them
// compile to global_* instructions. Through a generic pointer (one read from
// a table in memory, or chosen between two) they are flat instructions, which
// also count against the LDS wait counter, so every wait for an LDS result
// would also wait for them.
#define NHS_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ NHS_GLOBAL T* to_global(T* p) {
  return (NHS_GLOBAL T*)p;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;  // round to nearest even
  const uint32_t quiet_nan = (u >> 16) | 0x40u;
  // a select, not a branch, so that unrolled conversions stay straight-line
  return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? quiet_nan : rounded);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Scalar load/store of one element with a runtime dtype (used for queries
// and outputs, which are touched once per workgroup).
__device__ __forceinline__ float load_elem(const void* p, int dtype, int64_t i) {
  if (dtype == NHS_F32) return static_cast<const float*>(p)[i];
  uint32_t bits = static_cast<const uint16_t*>(p)[i];
  return dtype == NHS_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
}

__device__ __forceinline__ void store_elem(void* p, int dtype, int64_t i, float v) {
  if (dtype == NHS_F32) {
    static_cast<float*>(p)[i] = v;
  } else {
    static_cast<uint16_t*>(p)[i] = dtype == NHS_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
  }
}

// Storage tags for templated kernels.
struct F32 { static constexpr int dtype = NHS_F32; static constexpr int bytes = 4; };
struct F16 { static constexpr int dtype = NHS_F16; static constexpr int bytes = 2; };
struct BF16 { static constexpr int dtype = NHS_BF16; static constexpr int bytes = 2; };

// Loads E consecutive elements (E*bytes <= 16, naturally aligned) and
// converts them to fp32.
template <typename T, int E>
__device__ __forceinline__ void load_vec(const void* base, int64_t elem_index, float (&out)[E]) {
  constexpr int nbytes = E * T::bytes;
  const char* p = static_cast<const char*>(base) + elem_index * T::bytes;
  uint32_t w[(nbytes + 3) / 4];
  if constexpr (nbytes == 32) {
    const uint4 v0 = *reinterpret_cast<const uint4*>(p);
    const uint4 v1 = *reinterpret_cast<const uint4*>(p + 16);
    w[0] = v0.x; w[1] = v0.y; w[2] = v0.z; w[3] = v0.w;
    w[4] = v1.x; w[5] = v1.y; w[6] = v1.z; w[7] = v1.w;
  } else if constexpr (nbytes == 16) {
    uint4 v = *reinterpret_cast<const uint4*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (nbytes == 8) {
    uint2 v = *reinterpret_cast<const uint2*>(p);
    w[0] = v.x; w[1] = v.y;
  } else if constexpr (nbytes == 4) {
    w[0] = *reinterpret_cast<const uint32_t*>(p);
  } else {
    w[0] = *reinterpret_cast<const uint16_t*>(p);
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    if constexpr (T::dtype == NHS_F32) {
      out[e] = __uint_as_float(w[e]);
    } else {
      uint32_t half = (w[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
      out[e] = T::dtype == NHS_BF16 ? bf16_bits_to_f32(half) : f16_bits_to_f32(half);
    }
  }
}

// ---- wave64 cross-lane sums --------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of `lanes` lanes (a power of two <= 64); every
// lane of a group receives the group's sum. The additions form a pairwise
// tree in lane order: ((x0+x1)+(x2+x3))+((x4+x5)+(x6+x7)) ... so the result
// is bit-identical to tree_sum() of the CPU oracle.
__device__ __forceinline__ float group_sum(float x, int lanes) {
  if (lanes >= 2) x += dpp_f32<0xB1>(x);   // quad_perm [1,0,3,2]: partner lane ^ 1
  if (lanes >= 4) x += dpp_f32<0x4E>(x);   // quad_perm [2,3,0,1]: partner lane ^ 2
  if (lanes >= 8) x += dpp_f32<0x141>(x);  // row_half_mirror: quads swap within 8
  if (lanes >= 16) x += dpp_f32<0x140>(x); // row_mirror: halves swap within 16
  if (lanes >= 32) x += __shfl_xor(x, 16);
  if (lanes >= 64) x += __shfl_xor(x, 32);
  return x;
}

// ---- block-wide scans (blockDim.x a multiple of 64, <= 1024) -------------

// Exclusive prefix sum of `v` over the block in thread order. `scratch`
// needs blockDim.x / 64 + 1 elements. Returns the exclusive prefix; the
// block total is written to *total. Contains __syncthreads().
template <typename V>
__device__ V block_exclusive_scan(V v, V* scratch, V* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  V incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    V o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    V w = lane < nwaves ? scratch[lane] : V(0);
    V wi = w;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      V o = __shfl_up(wi, d);
      if (lane >= d) wi += o;
    }
    if (lane < nwaves) scratch[lane] = wi - w;  // exclusive wave offsets
    if (lane == nwaves - 1) scratch[nwaves] = wi;
  }
  __syncthreads();
  V result = scratch[wave] + incl - v;
  *total = scratch[nwaves];
  __syncthreads();
  return result;
}

template <typename V>
__device__ V block_sum(V v, V* scratch) {
  V total;
  block_exclusive_scan(v, scratch, &total);
  return total;
}

}  // namespace nhs
