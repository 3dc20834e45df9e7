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
//
// Two epilogues fuse the elementwise stage that follows a projection in the
// decode layer. Their tiles pair rows: tile rows 0-7 are weight rows
// base .. base + 7 and tile rows 8-15 are base + half .. base + half + 7, so
// each output element meets its partner in the same workgroup. Each row's
// fp32 sum is formed exactly as in the plain kernel (same K slices, same
// wave order), rounded as the plain kernel rounds it, and the elementwise
// stage then repeats the rounding steps of the launch it replaces
// (dense.hip): the outputs are bit-identical to the two launches.
//   silu-mul: w is a fused [gate; up] weight (2 * inter rows); tile t pairs
//     gate rows 8t .. 8t + 7 with up rows inter + 8t .. and writes
//     y[m, 8t + i] = round(round(silu(g)) * u).
//   rope: tile t of head h = t / (head_dim / 16) pairs dims 8j .. 8j + 7
//     with head_dim / 2 + 8j .. (j = t mod head_dim / 16) and rotates the
//     pair for heads below rope_heads.
#include "nhs_common.h"

namespace nhs {

constexpr int kLinMinWaves = 8, kLinMaxWaves = 16;  // waves per workgroup: K slices
enum { kEpiPlain = 0, kEpiSiluMul = 1, kEpiRope = 2 };

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
  // paired epilogues: tile t's base row is (t / per) * group_stride + (t % per) * 8
  int per, half;
  int64_t group_stride;
  int rope_tiles;            // tiles of the heads that rotate (rope)
  const char* cos;           // [m, cs_len] (rope)
  const char* sin;
  int cs_len;
};

template <typename T>
__device__ __forceinline__ float lin_round(float v) {
  return T::dtype == NHS_BF16 ? bf16_bits_to_f32(f32_to_bf16_bits(v)) : f16_bits_to_f32(f32_to_f16_bits(v));
}

// Weight rows are read as 512-byte row segments (two rows per load
// instruction, whole cache lines), written to the wave's own LDS region and
// read back in the MFMA operand layout: loaded straight in that layout a
// load instruction would cover 16 rows x 64 bytes, which streams at ~4.3
// TB/s against ~5.6 TB/s for long row segments. The region is private to
// the wave and LDS executes a wave's operations in order, so no barrier is
// needed between the writes and the reads.
constexpr int kLinWindow = 256;                       // k elements staged per window (512 bytes of a row)
constexpr int kLinRowBytes = kLinWindow * 2 + 16;     // staged row pitch (padded)

template <typename T, int RT, int EPI>
__global__ __launch_bounds__(kLinMaxWaves * kWave) void linear_small_m_kernel(LinearArgs a) {
  static_assert(EPI == kEpiPlain || RT == 1, "paired epilogues take one row tile");
  // dynamic LDS: each wave's staged rows, then the partial tiles [waves][RT][64 * 4]
  extern __shared__ __attribute__((aligned(16))) char lin_lds[];
  const int waves = (int)(blockDim.x >> 6);
  float* red = reinterpret_cast<float*>(lin_lds + (size_t)waves * RT * 16 * kLinRowBytes);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  char* stage = lin_lds + (size_t)wave * RT * 16 * kLinRowBytes;  // this wave's [RT * 16 rows][512 B]
  const int n0 = EPI == kEpiPlain ? (int)blockIdx.x * RT * 16
                                  : (int)(blockIdx.x / a.per) * (int)a.group_stride + (int)(blockIdx.x % a.per) * 8;
  const int row = lane & 15, kq = (lane >> 4) * 8;  // MFMA operand row and element offset
  const int slice = a.k / waves;                     // a multiple of kLinWindow
  const int k_begin = wave * slice;
  // tokens past m read row 0 and are zeroed (no branch between load and use)
  const bool live_tok = row < a.m;
  const char* xp = a.x + ((int64_t)(live_tok ? row : 0) * a.ldx + k_begin + kq) * T::bytes;
  // load mapping: instruction j covers tile rows 2j, 2j + 1 (lanes 0-31, 32-63), 16 bytes per lane
  const int lrow = lane >> 5, lcol = (lane & 31) * 16;
  const char* wrow = a.w + ((int64_t)(n0 + lrow) * a.ldw + k_begin) * T::bytes + lcol;
  // paired tiles: tile rows 8-15 (load instructions 4-7) sit half - 8 rows further
  const int64_t pair_skip = EPI == kEpiPlain ? 0 : (int64_t)(a.half - 8) * a.ldw;
  lin_f32x4 acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) acc[rt] = (lin_f32x4){0.f, 0.f, 0.f, 0.f};
  constexpr int kLoads = RT * 8;  // 16 rows per tile, two per instruction
  for (int w0 = 0; w0 < slice; w0 += kLinWindow) {
    uint4 wv[kLoads], xv[kLinWindow / 32];
#pragma unroll
    for (int j = 0; j < kLoads; ++j)
      wv[j] = *reinterpret_cast<const uint4*>(wrow + ((int64_t)(2 * j) * a.ldw + (j >= 4 ? pair_skip : 0) + w0) * T::bytes);
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
  if constexpr (EPI != kEpiPlain) {
#pragma clang fp contract(off)
    // D lane l < 32 holds tile rows (l / 16) * 4 + i < 8; lane l + 32 holds
    // their partners 8 rows down, kTile / 2 floats further in each tile
    const int t = (int)threadIdx.x;
    if (t >= kTile / 2) return;
    const int l = t >> 2, i = t & 3, tok = l & 15;
    if (tok >= a.m) return;
    const int rho = (l >> 4) * 4 + i;
    float lo = red[t], hi = red[t + kTile / 2];
    for (int w = 1; w < waves; ++w) {
      lo += red[w * kTile + t];
      hi += red[w * kTile + t + kTile / 2];
    }
    const int n_lo = n0 + rho, n_hi = n0 + a.half + rho;
    if (a.bias) {
      lo += load_elem(a.bias, T::dtype, n_lo);
      hi += load_elem(a.bias, T::dtype, n_hi);
    }
    lo = lin_round<T>(lo);  // the projection's output, as the plain kernel stores it
    hi = lin_round<T>(hi);
    if constexpr (EPI == kEpiSiluMul) {
      const float sg = lin_round<T>(lo / (1.0f + expf(-lo)));
      store_elem(a.y, T::dtype, (int64_t)tok * a.ldy + (int64_t)blockIdx.x * 8 + rho, sg * hi);
    } else {
      float y_lo = lo, y_hi = hi;
      if ((int)blockIdx.x < a.rope_tiles) {
        const int d = (int)(blockIdx.x % a.per) * 8 + rho;
        const float c = load_elem(a.cos, T::dtype, (int64_t)tok * a.cs_len + d);
        const float sn = load_elem(a.sin, T::dtype, (int64_t)tok * a.cs_len + d);
        y_lo = lin_round<T>(lo * c) + lin_round<T>(-hi * sn);
        y_hi = lin_round<T>(hi * c) + lin_round<T>(lo * sn);
      }
      store_elem(a.y, T::dtype, (int64_t)tok * a.ldy + n_lo, y_lo);
      store_elem(a.y, T::dtype, (int64_t)tok * a.ldy + n_hi, y_hi);
    }
    return;
  }
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

namespace nhs {

// Waves per workgroup: the most K slices (8..16) that divide the windows and
// leave every wave at least two (more loads in flight when the grid is
// small, e.g. 14 for k = 14336).
static int linear_waves(int k) {
  const int windows = k / kLinWindow;
  for (int w = kLinMaxWaves; w > kLinMinWaves; --w)
    if (windows % w == 0 && windows / w >= 2) return w;
  return kLinMinWaves;
}

static int check_linear(const char* who, const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride,
                        const void* y, int32_t dtype, int32_t m, int32_t k) {
  if (!x || !w || !y) return fail(NHS_ERR_INVALID, "%s: null pointer", who);
  if (dtype != NHS_BF16 && dtype != NHS_F16) return fail(NHS_ERR_UNSUPPORTED, "%s: bf16 or fp16 only", who);
  if (m < 1 || m > 16 || k < 1) return fail(NHS_ERR_INVALID, "%s: needs 1 <= m <= 16", who);
  if (k % (kLinMinWaves * kLinWindow))
    return fail(NHS_ERR_UNSUPPORTED, "%s: k must be a multiple of %d", who, kLinMinWaves * kLinWindow);
  if (x_row_stride < k || w_row_stride < k || x_row_stride % 8 || w_row_stride % 8)
    return fail(NHS_ERR_INVALID, "%s: bad row strides", who);
  if (((uintptr_t)x | (uintptr_t)w) % 16) return fail(NHS_ERR_INVALID, "%s: x and w must be 16-byte aligned", who);
  return 0;
}

template <int EPI>
static int launch_linear(const char* who, const LaunchEvents& ev, LinearArgs a, int32_t dtype, int tiles,
                         void* stream) {
  const int waves = linear_waves(a.k);
  const dim3 grid((unsigned)tiles), block((unsigned)(waves * kWave));
  const size_t lds = (size_t)waves * 16 * kLinRowBytes + (size_t)waves * kWave * 4 * sizeof(float);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == NHS_BF16)
    launch(linear_small_m_kernel<BF16, 1, EPI>, grid, block, lds, s, ev.start, ev.stop, a);
  else
    launch(linear_small_m_kernel<F16, 1, EPI>, grid, block, lds, s, ev.start, ev.stop, a);
  return launch_status(who);
}

static LinearArgs linear_args(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride,
                              const void* bias, int32_t m, int32_t n, int32_t k, void* y, int64_t y_row_stride) {
  LinearArgs a = {};
  a.x = static_cast<const char*>(x);
  a.w = static_cast<const char*>(w);
  a.bias = static_cast<const char*>(bias);
  a.y = static_cast<char*>(y);
  a.ldx = x_row_stride, a.ldw = w_row_stride, a.ldy = y_row_stride;
  a.m = m, a.n = n, a.k = k;
  return a;
}

}  // namespace nhs

extern "C" int nhs_linear_small_m(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride,
                                  const void* bias, int32_t dtype, int32_t m, int32_t n, int32_t k, void* y,
                                  int64_t y_row_stride, void* stream) {
  using namespace nhs;
  const LaunchEvents ev = take_launch_events();
  const char* who = "nhs_linear_small_m";
  if (int st = check_linear(who, x, x_row_stride, w, w_row_stride, y, dtype, m, k)) return st;
  if (n < 16 || n % 16) return fail(NHS_ERR_UNSUPPORTED, "%s: n must be a multiple of 16", who);
  if (y_row_stride < n) return fail(NHS_ERR_INVALID, "%s: bad row strides", who);
  const LinearArgs a = linear_args(x, x_row_stride, w, w_row_stride, bias, m, n, k, y, y_row_stride);
  return launch_linear<kEpiPlain>(who, ev, a, dtype, n / 16, stream);
}

extern "C" int nhs_linear_silu_mul(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride,
                                   int32_t dtype, int32_t m, int32_t inter, int32_t k, void* y, int64_t y_row_stride,
                                   void* stream) {
  using namespace nhs;
  const LaunchEvents ev = take_launch_events();
  const char* who = "nhs_linear_silu_mul";
  if (int st = check_linear(who, x, x_row_stride, w, w_row_stride, y, dtype, m, k)) return st;
  if (inter < 8 || inter % 8)
    return fail(NHS_ERR_UNSUPPORTED, "%s: inter must be a multiple of 8", who);
  if (y_row_stride < inter) return fail(NHS_ERR_INVALID, "%s: bad row strides", who);
  LinearArgs a = linear_args(x, x_row_stride, w, w_row_stride, nullptr, m, 2 * inter, k, y, y_row_stride);
  a.per = inter / 8, a.half = inter, a.group_stride = 0;
  return launch_linear<kEpiSiluMul>(who, ev, a, dtype, inter / 8, stream);
}

extern "C" int nhs_linear_rope(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride,
                               const void* bias, int32_t dtype, int32_t m, int32_t n, int32_t k, int32_t head_dim,
                               int32_t rope_heads, const void* cos, const void* sin, void* y, int64_t y_row_stride,
                               void* stream) {
  using namespace nhs;
  const LaunchEvents ev = take_launch_events();
  const char* who = "nhs_linear_rope";
  if (int st = check_linear(who, x, x_row_stride, w, w_row_stride, y, dtype, m, k)) return st;
  if (head_dim < 16 || head_dim % 16 || n < head_dim || n % head_dim)
    return fail(NHS_ERR_UNSUPPORTED, "%s: head_dim must be a multiple of 16 and n a multiple of head_dim", who);
  if (rope_heads < 0 || (int64_t)rope_heads * head_dim > n)
    return fail(NHS_ERR_INVALID, "%s: rope_heads beyond the row's heads", who);
  if (rope_heads > 0 && (!cos || !sin)) return fail(NHS_ERR_INVALID, "%s: null cos/sin", who);
  if (y_row_stride < n) return fail(NHS_ERR_INVALID, "%s: bad row strides", who);
  LinearArgs a = linear_args(x, x_row_stride, w, w_row_stride, bias, m, n, k, y, y_row_stride);
  a.per = head_dim / 16, a.half = head_dim / 2, a.group_stride = head_dim;
  a.rope_tiles = rope_heads * a.per;
  a.cos = static_cast<const char*>(cos), a.sin = static_cast<const char*>(sin), a.cs_len = head_dim / 2;
  return launch_linear<kEpiRope>(who, ev, a, dtype, n / 16, stream);
}
