// Linear layer for a handful of token rows (decode): y[m, n] = sum_k x[m, k]
// * w[n, k] (+ bias[n]), m < 16, bf16 or fp16 in and out, fp32 accumulation.
//
// At decode batch sizes the product is a stream of the weight matrix (2
// bytes per weight, 16 flops or fewer), so the kernel is built to read the
// weights at the HBM rate: a workgroup of W waves (8..16) owns a tile of 16
// weight rows and the full K; wave w takes the K slice [w K/W, (w+1) K/W) and walks
// it in windows of 256 k, 32-wide steps with v_mfma_f32_16x16x32, the
// weight rows as the A operand (lane l: row l % 16, elements (l / 16) * 8
// .. +7 of the step) and the token rows as the B operand (lane l: token
// l % 16, the same elements; tokens past m read as zero). The W partial
// tiles are added through LDS in wave order, the bias is added in fp32 and
// the sum is rounded once.
#include "nhs_common.h"

namespace nhs {

constexpr int kLinMinWaves = 8, kLinMaxWaves = 16;  // waves per workgroup: K slices

typedef __bf16 lin_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 lin_f16x8 __attribute__((ext_vector_type(8)));
typedef float lin_f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ lin_f32x4 lin_mfma(uint4 a, uint4 b, lin_f32x4 c) {
  if constexpr (T::dtype == NHS_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(lin_bf16x8, a), __builtin_bit_cast(lin_bf16x8, b),
                                                  c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(lin_f16x8, a), __builtin_bit_cast(lin_f16x8, b), c,
                                                 0, 0, 0);
}

struct LinearArgs {
  const char* x;
  const char* w;
  const char* bias;  // may be null
  char* y;
  int64_t ldx, ldw, ldy;  // row strides in elements
  int m, n, k;
};

// Weight rows are read as 512-byte row segments (two rows per load
// instruction, whole cache lines), written to the wave's own LDS region and
// read back in the MFMA operand layout: loaded straight in that layout a
// load instruction would cover 16 rows x 64 bytes, which streams at ~4.3
// TB/s against ~5.6 TB/s for long row segments. The region is private to
// the wave and LDS executes a wave's operations in order, so no barrier is
// needed between the writes and the reads.
constexpr int kLinWindow = 256;                       // k elements staged per window (512 bytes of a row)
constexpr int kLinRowBytes = kLinWindow * 2 + 16;     // staged row pitch (padded)

template <typename T, int RT>
__global__ __launch_bounds__(kLinMaxWaves * kWave) void linear_small_m_kernel(LinearArgs a) {
  // dynamic LDS: each wave's staged rows, then the partial tiles [waves][RT][64 * 4]
  extern __shared__ __attribute__((aligned(16))) char lin_lds[];
  const int waves = (int)(blockDim.x >> 6);
  float* red = reinterpret_cast<float*>(lin_lds + (size_t)waves * RT * 16 * kLinRowBytes);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  char* stage = lin_lds + (size_t)wave * RT * 16 * kLinRowBytes;  // this wave's [RT * 16 rows][512 B]
  const int n0 = blockIdx.x * RT * 16;
  const int row = lane & 15, kq = (lane >> 4) * 8;  // MFMA operand row and element offset
  const int slice = a.k / waves;                     // a multiple of kLinWindow
  const int k_begin = wave * slice;
  // tokens past m read row 0 and are zeroed (no branch between load and use)
  const bool live_tok = row < a.m;
  const char* xp = a.x + ((int64_t)(live_tok ? row : 0) * a.ldx + k_begin + kq) * T::bytes;
  // load mapping: instruction j covers tile rows 2j, 2j + 1 (lanes 0-31, 32-63), 16 bytes per lane
  const int lrow = lane >> 5, lcol = (lane & 31) * 16;
  const char* wrow = a.w + ((int64_t)(n0 + lrow) * a.ldw + k_begin) * T::bytes + lcol;
  lin_f32x4 acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) acc[rt] = (lin_f32x4){0.f, 0.f, 0.f, 0.f};
  constexpr int kLoads = RT * 8;  // 16 rows per tile, two per instruction
  for (int w0 = 0; w0 < slice; w0 += kLinWindow) {
    uint4 wv[kLoads], xv[kLinWindow / 32];
#pragma unroll
    for (int j = 0; j < kLoads; ++j)
      wv[j] = *reinterpret_cast<const uint4*>(wrow + ((int64_t)(2 * j) * a.ldw + w0) * T::bytes);
#pragma unroll
    for (int s = 0; s < kLinWindow / 32; ++s)
      xv[s] = *reinterpret_cast<const uint4*>(xp + (int64_t)(w0 + s * 32) * T::bytes);
#pragma unroll
    for (int j = 0; j < kLoads; ++j)
      *reinterpret_cast<uint4*>(stage + (2 * j + lrow) * kLinRowBytes + lcol) = wv[j];
#pragma unroll
    for (int s = 0; s < kLinWindow / 32; ++s) {
      const uint4 xb = live_tok ? xv[s] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const uint4 wa = *reinterpret_cast<const uint4*>(stage + (rt * 16 + row) * kLinRowBytes + (s * 32 + kq) * 2);
        acc[rt] = lin_mfma<T>(wa, xb, acc[rt]);
      }
    }
  }
  constexpr int kTile = kWave * 4;  // partial tile floats per wave and row tile
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
    *reinterpret_cast<float4*>(&red[(wave * RT + rt) * kTile + lane * 4]) =
        make_float4(acc[rt][0], acc[rt][1], acc[rt][2], acc[rt][3]);
  __syncthreads();
  // D lane l holds weight rows (l / 16) * 4 + i of the tile, token l % 16
  for (int t = threadIdx.x; t < RT * kTile; t += (int)blockDim.x) {
    const int rt = t / kTile, r = t - rt * kTile;
    const int l = r >> 2, i = r & 3;
    const int tok = l & 15;
    if (tok >= a.m) continue;
    float v = red[rt * kTile + r];
    for (int w = 1; w < waves; ++w) v += red[(w * RT + rt) * kTile + r];
    const int n = n0 + rt * 16 + (l >> 4) * 4 + i;
    if (a.bias) v += load_elem(a.bias, T::dtype, n);
    store_elem(a.y, T::dtype, (int64_t)tok * a.ldy + n, v);
  }
}

}  // namespace nhs

extern "C" int nhs_linear_small_m(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride,
                                  const void* bias, int32_t dtype, int32_t m, int32_t n, int32_t k, void* y,
                                  int64_t y_row_stride, void* stream) {
  using namespace nhs;
  const LaunchEvents ev = take_launch_events();
  const char* who = "nhs_linear_small_m";
  if (!x || !w || !y) return fail(NHS_ERR_INVALID, "%s: null pointer", who);
  if (dtype != NHS_BF16 && dtype != NHS_F16) return fail(NHS_ERR_UNSUPPORTED, "%s: bf16 or fp16 only", who);
  if (m < 1 || m > 16 || n < 16 || k < 1) return fail(NHS_ERR_INVALID, "%s: needs 1 <= m <= 16, n >= 16", who);
  if (n % 16 || k % (kLinMinWaves * kLinWindow))
    return fail(NHS_ERR_UNSUPPORTED, "%s: n must be a multiple of 16 and k of %d", who, kLinMinWaves * kLinWindow);
  if (x_row_stride < k || w_row_stride < k || y_row_stride < n || x_row_stride % 8 || w_row_stride % 8)
    return fail(NHS_ERR_INVALID, "%s: bad row strides", who);
  if (((uintptr_t)x | (uintptr_t)w) % 16) return fail(NHS_ERR_INVALID, "%s: x and w must be 16-byte aligned", who);
  LinearArgs a;
  a.x = static_cast<const char*>(x);
  a.w = static_cast<const char*>(w);
  a.bias = static_cast<const char*>(bias);
  a.y = static_cast<char*>(y);
  a.ldx = x_row_stride, a.ldw = w_row_stride, a.ldy = y_row_stride;
  a.m = m, a.n = n, a.k = k;
  hipStream_t s = (hipStream_t)stream;
  // waves per workgroup: the most K slices (8..16) that divide the windows
  // and leave every wave at least two (more loads in flight when the grid
  // is small, e.g. 14 for k = 14336)
  const int windows = k / kLinWindow;
  int waves = kLinMinWaves;
  for (int w = kLinMaxWaves; w > kLinMinWaves; --w)
    if (windows % w == 0 && windows / w >= 2) {
      waves = w;
      break;
    }
  const dim3 grid((unsigned)(n / 16)), block((unsigned)(waves * kWave));
  const size_t lds = (size_t)waves * 16 * kLinRowBytes + (size_t)waves * kWave * 4 * sizeof(float);
  if (dtype == NHS_BF16)
    launch(linear_small_m_kernel<BF16, 1>, grid, block, lds, s, ev.start, ev.stop, a);
  else
    launch(linear_small_m_kernel<F16, 1>, grid, block, lds, s, ev.start, ev.stop, a);
  return launch_status(who);
}
