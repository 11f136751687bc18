// Reference-format kernels: e4m3fn codecs, per-row FP8 dequant, signed-nibble
// int4 dequant, and the float32 Linear forward on those formats.
//
// These reproduce python/ccut/quant/kernels.py bit for bit (dequant, codecs)
// and quant/weight_only.py / quant/method.py within float32 summation order
// (the matmuls).  All are HBM-bound streaming kernels.
#include "ccq_common.h"

#include <math.h>

namespace ccq {

// float -> e4m3fn with the reference's rounding: round-half-UP on the
// magnitude, |v| >= 464 -> 0x7E, NaN -> 0x7F, sign only for v < 0
// (kernels.py:77-123).  Works on the bit pattern so that it does not depend
// on the denormal mode of the float pipeline.
__device__ __forceinline__ uint32_t f32_to_fp8_halfup(float v) {
  uint32_t u = __float_as_uint(v);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return 0x7Fu;                       // NaN
  if (a == 0) return 0u;                                   // +0 and -0 -> 0x00
  uint32_t sign = (u >> 24) & 0x80u;
  if (a >= 0x43e80000u) return sign | 0x7Eu;               // >= 464
  if (a < 0x3c800000u) {                                   // < 2^-6
    if ((a >> 23) == 0) return sign;                       // f32 denormal: rounds to 0
    float t = __uint_as_float(a) * 512.0f;                 // exact
    float fl = floorf(t);
    uint32_t m = (uint32_t)fl + ((t - fl) >= 0.5f ? 1u : 0u);
    return sign | (m >= 8u ? 0x08u : m);
  }
  int e = (int)(a >> 23) - 127;                            // floor(log2 v), exact
  float m = __uint_as_float((a & 0x007fffffu) | (127u << 23)) - 1.0f;  // v*2^-e - 1, exact
  float t = m * 8.0f;                                      // exact
  float fl = floorf(t);
  uint32_t mant = (uint32_t)fl + ((t - fl) >= 0.5f ? 1u : 0u);
  int ec = e + 7;
  if (mant >= 8u) {
    mant = 0;
    ec += 1;
  }
  if (ec >= 15 && mant > 6u) mant = 6;
  return sign | (((uint32_t)ec & 0xFu) << 3) | mant;
}

__global__ void fp8_to_f32_kernel(const uint8_t* __restrict__ code, float* __restrict__ out, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) out[i] = fp8_e4m3_to_f32(code[i]);
}

__global__ void f32_to_fp8_kernel(const float* __restrict__ x, uint8_t* __restrict__ out, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) out[i] = (uint8_t)f32_to_fp8_halfup(x[i]);
}

// out[r, c] = fp8(w[r, c]) * scale[r]; one float32 multiply of two exact
// operands = the reference's float64 product rounded once to float32.
__global__ void fp8_dequant_kernel(const uint8_t* __restrict__ w, const float* __restrict__ scale,
                                   float* __restrict__ out, int64_t rows, int64_t cols) {
  int64_t n = rows * cols;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    int64_t r = i / cols;
    out[i] = fp8_e4m3_to_f32(w[i]) * scale[r];
  }
}

__device__ __forceinline__ float nib_signed(uint32_t v) {
  int q = (int)(v & 0xFu);
  return (float)(q >= 8 ? q - 16 : q);
}

// NF4 code -> value: table[code] for code < table_len; past the table NaN
// (the reference indexes its 8-entry table with the 4-bit code unchecked,
// kernels.py:299-322, an out-of-bounds read for codes 8..15)
__device__ __forceinline__ float nf4_val(uint32_t v, const float* __restrict__ table, int table_len) {
  const int q = (int)(v & 0xFu);
  return q < table_len ? table[q] : __int_as_float(0x7fc00000);
}

__global__ void nf4_dequant_kernel(const uint8_t* __restrict__ packed, const float* __restrict__ scale,
                                   const float* __restrict__ table, int table_len, float* __restrict__ out,
                                   int64_t rows, int64_t cols) {
  const int64_t half = cols / 2, n = rows * half;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    const int64_t r = i / half, j = i - r * half;
    const uint32_t b = packed[i];
    out[r * cols + 2 * j] = nf4_val(b, table, table_len) * scale[2 * j];
    out[r * cols + 2 * j + 1] = nf4_val(b >> 4, table, table_len) * scale[2 * j + 1];
  }
}

// int8_quantize_row (kernels.py:192-211): per column c, inv = 127 / amax[c]
// in float64 (0 when amax[c] is not > 0), q = round-half-even(x * inv) in
// float64, clamped to +-127.  The reference leaves NaN and +-inf products
// undefined (numba fastmath, int() of a non-finite float); here NaN -> 0,
// +-inf -> +-127.
__global__ void int8_quantize_cols_kernel(const float* __restrict__ x, const float* __restrict__ amax,
                                          int8_t* __restrict__ out, int64_t rows, int64_t cols) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < rows * cols; i += stride) {
    const float a = amax[i % cols];
    const double inv = a > 0.f ? 127.0 / (double)a : 0.0;
    const double q = rint((double)x[i] * inv);
    out[i] = q != q ? (int8_t)0 : (int8_t)(int)fmin(fmax(q, -127.0), 127.0);
  }
}

// packed [rows, cols/2]: byte j -> columns 2j (low nibble), 2j+1 (high).
__global__ void int4_dequant_kernel(const uint8_t* __restrict__ packed, const float* __restrict__ scale,
                                    float* __restrict__ out, int64_t rows, int64_t cols) {
  int64_t half = cols / 2;
  int64_t n = rows * half;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    int64_t r = i / half, j = i - r * half;
    uint32_t b = packed[i];
    out[r * cols + 2 * j] = nib_signed(b) * scale[2 * j];
    out[r * cols + 2 * j + 1] = nib_signed(b >> 4) * scale[2 * j + 1];
  }
}

// ----------------------------------------------------------------------------
// float32 Linear on the reference formats: y[b, r] = sum_c x[b, c] * W[r, c].
// One wave per output row r (the row of W is contiguous), BB batch rows per
// pass with the weight element dequantized once per pass.  W elements are
// formed exactly as the dequant kernels above, then FMA-accumulated in fp32.
// ----------------------------------------------------------------------------
constexpr int kLinBB = 8;

// kFmt: 0 int4 or 3 NF4 (two codes per byte, scale per input column), 1 fp8
// e4m3 or 2 int8 (one code per byte, scale per output row)
template <int kFmt>
__global__ __launch_bounds__(256) void ref_linear_f32_kernel(const float* __restrict__ x,
                                                             const uint8_t* __restrict__ w,
                                                             const float* __restrict__ scale,
                                                             float* __restrict__ y, int64_t batch,
                                                             int64_t in_f, int64_t out_f,
                                                             const float* __restrict__ table, int table_len) {
  const int lane = lane_id();
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= out_f) return;
  const int64_t b0 = (int64_t)blockIdx.y * kLinBB;
  const int nb = (int)min<int64_t>(kLinBB, batch - b0);
  constexpr bool kByte = kFmt == 1 || kFmt == 2;
  const int64_t row_bytes = kByte ? in_f : in_f / 2;
  const uint8_t* wr = w + r * row_bytes;
  float acc[kLinBB];
#pragma unroll
  for (int b = 0; b < kLinBB; ++b) acc[b] = 0.f;
  for (int64_t byte = lane; byte < row_bytes; byte += 64) {
    uint32_t v = wr[byte];
    if (kByte) {
      // W[r,c] as fp8_dequant_mat / int8_dequant_row form it
      const float wv = (kFmt == 1 ? fp8_e4m3_to_f32(v) : (float)(int8_t)v) * scale[r];
      const int64_t c = byte;
#pragma unroll
      for (int b = 0; b < kLinBB; ++b)
        if (b < nb) acc[b] = fmaf(x[(b0 + b) * in_f + c], wv, acc[b]);
    } else {
      const int64_t c = 2 * byte;
      float w0 = (kFmt == 3 ? nf4_val(v, table, table_len) : nib_signed(v)) * scale[c];
      float w1 = (kFmt == 3 ? nf4_val(v >> 4, table, table_len) : nib_signed(v >> 4)) * scale[c + 1];
#pragma unroll
      for (int b = 0; b < kLinBB; ++b)
        if (b < nb) {
          const float* xr = x + (b0 + b) * in_f + c;
          acc[b] = fmaf(xr[0], w0, acc[b]);
          acc[b] = fmaf(xr[1], w1, acc[b]);
        }
    }
  }
#pragma unroll
  for (int b = 0; b < kLinBB; ++b) {
    float v = acc[b];
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    acc[b] = v;
  }
  if (lane == 0)
    for (int b = 0; b < nb; ++b) y[(b0 + b) * out_f + r] = acc[b];
}

// The same Linear for the byte formats (fp8 e4m3, int8; one scale per output
// row) and int4 (one scale per input column), streaming W in 16-byte pieces.
// A workgroup is 4 waves x RT output rows; lane l of a wave takes bytes
// 16 l + 1024 i of each of its rows (all RT rows at once, so every lane
// reads its piece of x once per RT rows), BB batch rows per pass from x
// staged in LDS (int4: x[c] * s[c] staged, the column scale taken out of
// the sum; fp8/int8: the row scale applied to the row's sum).  fp8 codes
// decode with the hardware converter (v_cvt_pk_f32_fp8: e4m3fn, exact,
// NaN for 0x7F / 0xFF as fp8_e4m3_to_f32 above).  Sums are float32 FMAs,
// in a different order from ref_linear_f32_kernel.
// rows per wave: 8 for passes of 2+ batch rows (halves the x reads per
// weight; measured 46 -> 26 us at 4 x 4096 x 14336), 4 for single rows (more
// waves for small N)
template <int BB>
constexpr int rv_rows() { return BB == 1 ? 4 : 8; }
constexpr int RV_LDS = 64 * 1024;     // staged x bytes per workgroup at most

// Sums over the wave of V values per lane (V a power of two <= 64): halving
// exchanges (V - 1 shuffles), then whole-value ones; lane l ends with the
// sum of value l & (V - 1), in a fixed order.
template <int V>
__device__ __forceinline__ float wave_reduce_scatter(float (&v)[V], int lane) {
#pragma unroll
  for (int m = 1, n = V; m < V; m <<= 1, n >>= 1) {
    const bool up = (lane & m) != 0;
#pragma unroll
    for (int j = 0; j < n / 2; ++j) {
      const float keep = up ? v[2 * j + 1] : v[2 * j];
      const float send = up ? v[2 * j] : v[2 * j + 1];
      v[j] = keep + __shfl_xor(send, m, 64);
    }
  }
  float t = v[0];
#pragma unroll
  for (int m = V; m < 64; m <<= 1) t += __shfl_xor(t, m, 64);
  return t;
}

template <int kFmt, int BB>
__global__ __launch_bounds__(256) void ref_linear_vec_kernel(const float* __restrict__ x,
                                                             const uint8_t* __restrict__ w,
                                                             const float* __restrict__ scale,
                                                             float* __restrict__ y, int64_t batch,
                                                             int64_t in_f, int64_t out_f) {
  extern __shared__ __align__(16) float xs[];  // [BB][in_f]
  constexpr bool kNib = kFmt == 0;
  constexpr int RV_RT = rv_rows<BB>();
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b0 = (int64_t)blockIdx.y * BB;
  const int nb = (int)min<int64_t>(BB, batch - b0);
  // x rows of this pass (rows past the batch: zeros), int4 with the column
  // scale; 16 bytes per thread and copy, 8 copies in flight per thread
  const int q4 = (int)(in_f / 4), nq = BB * q4;  // 16-byte pieces per row, per pass
  for (int i0 = 0; i0 < nq; i0 += 8 * 256) {
    f32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * 256 + tid, b = i / q4, c4 = i - b * q4;
      v[u] = i < nq && b < nb ? *reinterpret_cast<const f32x4*>(x + (b0 + b) * in_f + 4 * c4)
                              : f32x4{0.f, 0.f, 0.f, 0.f};
      if (kNib && i < nq) {
        const f32x4 sc = *reinterpret_cast<const f32x4*>(scale + 4 * c4);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[u][e] *= sc[e];
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * 256 + tid;
      if (i < nq) *reinterpret_cast<f32x4*>(&xs[4 * i]) = v[u];
    }
  }
  __syncthreads();
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * RV_RT;
  if (row0 >= out_f) return;
  const int64_t row_bytes = kNib ? in_f / 2 : in_f;  // a multiple of 16
  const uint8_t* wr[RV_RT];
#pragma unroll
  for (int r = 0; r < RV_RT; ++r) wr[r] = w + min(row0 + r, out_f - 1) * row_bytes;  // past the end: the last row, not stored
  float acc[RV_RT][BB];
#pragma unroll
  for (int r = 0; r < RV_RT; ++r)
#pragma unroll
    for (int b = 0; b < BB; ++b) acc[r][b] = 0.f;
  for (int64_t off = (int64_t)lane * 16; off < row_bytes; off += 1024) {
    u32x4 q[RV_RT];
#pragma unroll
    for (int r = 0; r < RV_RT; ++r) q[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr[r] + off));
    constexpr int NE = kNib ? 32 : 16;  // elements per 16-byte piece
    const int64_t c0 = kNib ? 2 * off : off;
#pragma unroll
    for (int h = 0; h < NE / 8; ++h) {  // 8 elements (32 x bytes per batch row) at a time
      float xv[BB][8];
#pragma unroll
      for (int b = 0; b < BB; ++b) {
        const f32x4 lo = *reinterpret_cast<const f32x4*>(&xs[b * in_f + c0 + 8 * h]);
        const f32x4 hi = *reinterpret_cast<const f32x4*>(&xs[b * in_f + c0 + 8 * h + 4]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xv[b][e] = lo[e];
          xv[b][4 + e] = hi[e];
        }
      }
#pragma unroll
      for (int r = 0; r < RV_RT; ++r) {
        float wv[8];
        if constexpr (kFmt == 1) {  // fp8: bytes 8h .. 8h + 7 of the piece
#pragma unroll
          for (int d = 0; d < 2; ++d) {
            const uint32_t word = q[r][2 * h + d];
            const auto p0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)word, false);
            const auto p1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)word, true);
            wv[4 * d] = p0[0];
            wv[4 * d + 1] = p0[1];
            wv[4 * d + 2] = p1[0];
            wv[4 * d + 3] = p1[1];
          }
        } else if constexpr (kFmt == 2) {  // int8
#pragma unroll
          for (int e = 0; e < 8; ++e) wv[e] = (float)((int)(q[r][(8 * h + e) >> 2] << (24 - 8 * (e & 3))) >> 24);
        } else {  // int4: nibbles 8h .. 8h + 7 = word h, low nibble first (column 2j, 2j + 1 of byte j)
#pragma unroll
          for (int e = 0; e < 8; ++e) wv[e] = (float)((int)(q[r][h] << (28 - 4 * e)) >> 28);  // signed nibble
        }
#pragma unroll
        for (int b = 0; b < BB; ++b)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[r][b] = fmaf(xv[b][e], wv[e], acc[r][b]);
      }
    }
  }
  float flat[RV_RT * BB];
#pragma unroll
  for (int r = 0; r < RV_RT; ++r)
#pragma unroll
    for (int b = 0; b < BB; ++b) flat[r * BB + b] = acc[r][b];
  const float v = wave_reduce_scatter<RV_RT * BB>(flat, lane);
  if (lane < RV_RT * BB) {  // lane l: row l / BB, batch row l % BB
    const int r = lane / BB, b = lane % BB;
    const int64_t row = row0 + r;
    if (row < out_f && b < nb) y[(b0 + b) * out_f + row] = kNib ? v : v * scale[row];
  }
}

// out = g / (1 + exp(-g)) * u in float64, stored float32 (kernels.py:219-231)
// out[i] = s[i / G] for i < groups * G.
__global__ void group_broadcast_kernel(const float* __restrict__ s, float* __restrict__ out, int64_t n, int64_t G) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) out[i] = s[i / G];
}

__global__ void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ out,
                                int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    const double t = (double)g[i];
    out[i] = (float)((t / (1.0 + exp(-t))) * (double)u[i]);
  }
}

__global__ void zero_f32_kernel(float* __restrict__ y, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) y[i] = 0.f;
}

// |x| maximum of a row with numpy's NaN rule (any NaN gives NaN), over the
// 256 threads of a workgroup; every thread gets the result.
__device__ float row_amax_256(float m, bool nan, float* red) {
  for (int off = 32; off >= 1; off >>= 1) {
    m = fmaxf(m, __shfl_xor(m, off, 64));
    nan = __shfl_xor((int)nan, off, 64) != 0 || nan;
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = nan ? __builtin_nanf("") : m;
  __syncthreads();
  float a = red[0];
  for (int i = 1; i < 4; ++i) a = (a != a || red[i] != red[i]) ? __builtin_nanf("") : fmaxf(a, red[i]);
  __syncthreads();
  return a;
}

// np.clip(q, -448, 448) keeps NaN
__device__ __forceinline__ float clip448(float q) { return q != q ? q : fminf(fmaxf(q, -448.0f), 448.0f); }

// Load-time quantization of a BF16 [rows, cols] weight to e4m3 codes, one
// row per workgroup (quant/online.py:37-64): s = scale[r] when given, else
// amax / 448 in float64 (0 -> 1); s <= 0 or NaN -> 1; code =
// half-up(clip(w / float32(s), +-448)) with a float32 division, as numpy
// divides a float32 row by a Python float.
__global__ __launch_bounds__(256) void quant_rows_fp8_kernel(const uint16_t* __restrict__ w,
                                                             const float* __restrict__ scale,
                                                             uint8_t* __restrict__ out, int64_t cols) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const uint16_t* row = w + r * cols;
  float m = 0.f;
  bool nan = false;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    const float v = __uint_as_float((uint32_t)row[c] << 16);
    m = fmaxf(m, fabsf(v));
    nan = nan || v != v;
  }
  double s;
  if (scale != nullptr) {
    s = (double)scale[r];
  } else {
    s = (double)row_amax_256(m, nan, red) / 448.0;
    if (s == 0.0) s = 1.0;  // `amax / 448.0 or 1.0`: only 0.0 is falsy
  }
  if (!(s > 0.0)) s = 1.0;
  const float s32 = (float)s;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    const float v = __uint_as_float((uint32_t)row[c] << 16);
    out[r * cols + c] = (uint8_t)f32_to_fp8_halfup(clip448(v / s32));
  }
}

// Per-token KV quantization (quant/kv.py:70-90): one row (side, head,
// token) of `dim` float32 per workgroup; amax <= 0 -> codes and scale 0;
// else s = amax / 448 (float64), codes = half-up(clip(x / float32(s))),
// scale byte = half-up(float32(s)).  A NaN in the row gives NaN codes.
__global__ __launch_bounds__(256) void kv_quant_fp8_kernel(const float* __restrict__ kv, uint8_t* __restrict__ out,
                                                           uint8_t* __restrict__ scales, int64_t dim) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const float* row = kv + r * dim;
  float m = 0.f;
  bool nan = false;
  for (int64_t c = threadIdx.x; c < dim; c += blockDim.x) {
    const float v = row[c];
    m = fmaxf(m, fabsf(v));
    nan = nan || v != v;
  }
  const float amax = row_amax_256(m, nan, red);
  if (amax <= 0.f) {
    for (int64_t c = threadIdx.x; c < dim; c += blockDim.x) out[r * dim + c] = 0;
    if (threadIdx.x == 0) scales[r] = 0;
    return;
  }
  const float s32 = (float)((double)amax / 448.0);
  for (int64_t c = threadIdx.x; c < dim; c += blockDim.x)
    out[r * dim + c] = (uint8_t)f32_to_fp8_halfup(clip448(row[c] / s32));
  if (threadIdx.x == 0) scales[r] = (uint8_t)f32_to_fp8_halfup(s32);
}

// KV read-back (quant/kv.py:93-101): out = decode(code) * decode(scale)
// (float32 product) where the scale decodes to > 0, else 0.
__global__ void kv_dequant_fp8_kernel(const uint8_t* __restrict__ codes, const uint8_t* __restrict__ scales,
                                      float* __restrict__ out, int64_t n, int64_t dim) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    const float sc = fp8_e4m3_to_f32(scales[i / dim]);
    out[i] = sc > 0.f ? fp8_e4m3_to_f32(codes[i]) * sc : 0.f;
  }
}

// The same load-time quantization with 16-byte loads (cols % 8 == 0,
// cols <= 2048 * VPT): each thread keeps its VPT x 8 values in registers
// between the amax and the encode, and stores 8 codes at a time.
template <int VPT>
__global__ __launch_bounds__(256) void quant_rows_fp8_vec_kernel(const uint16_t* __restrict__ w,
                                                                 const float* __restrict__ scale,
                                                                 uint8_t* __restrict__ out, int64_t cols) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const u32x4* row = reinterpret_cast<const u32x4*>(w + r * cols);
  const int nv = (int)(cols / 8);
  float v[VPT][8];
  float m = 0.f;
  bool nan = false;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int idx = (int)threadIdx.x + 256 * j;
    if (idx < nv) {
      const u32x4 q = row[idx];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t word = q[e >> 1];
        v[j][e] = __uint_as_float((e & 1) ? (word & 0xffff0000u) : (word << 16));
        m = fmaxf(m, fabsf(v[j][e]));
        nan = nan || v[j][e] != v[j][e];
      }
    }
  }
  double s;
  if (scale != nullptr) {
    s = (double)scale[r];
  } else {
    s = (double)row_amax_256(m, nan, red) / 448.0;
    if (s == 0.0) s = 1.0;
  }
  if (!(s > 0.0)) s = 1.0;
  const float s32 = (float)s;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int idx = (int)threadIdx.x + 256 * j;
    if (idx < nv) {
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo |= f32_to_fp8_halfup(clip448(v[j][e] / s32)) << (8 * e);
        hi |= f32_to_fp8_halfup(clip448(v[j][4 + e] / s32)) << (8 * e);
      }
      reinterpret_cast<uint2*>(out + r * cols)[idx] = make_uint2(lo, hi);
    }
  }
}

// KV rows of dim <= 4 * TPR floats (dim % 4 == 0): TPR threads per row,
// 4 values each, the amax over the row's lanes by butterfly (TPR divides
// 64, so a row never spans two waves).
template <int TPR>
__device__ __forceinline__ float group_amax(float m, bool nan) {
#pragma unroll
  for (int off = TPR / 2; off >= 1; off >>= 1) {
    m = fmaxf(m, __shfl_xor(m, off, 64));
    nan = __shfl_xor((int)nan, off, 64) != 0 || nan;
  }
  return nan ? __builtin_nanf("") : m;
}

template <int TPR>
__global__ __launch_bounds__(256) void kv_quant_fp8_vec_kernel(const float* __restrict__ kv, uint8_t* __restrict__ out,
                                                               uint8_t* __restrict__ scales, int64_t rows,
                                                               int64_t dim) {
  const int64_t r = (int64_t)blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
  const int l = threadIdx.x % TPR, c = 4 * l;
  const bool ok = r < rows && c < dim;
  f32x4 x = f32x4{0.f, 0.f, 0.f, 0.f};
  if (ok) x = *reinterpret_cast<const f32x4*>(kv + r * dim + c);
  float m = 0.f;
  bool nan = false;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    m = fmaxf(m, fabsf(x[e]));
    nan = nan || x[e] != x[e];
  }
  const float amax = group_amax<TPR>(m, nan);
  if (r >= rows) return;
  if (amax <= 0.f) {
    if (ok) *reinterpret_cast<uint32_t*>(out + r * dim + c) = 0u;
    if (l == 0) scales[r] = 0;
    return;
  }
  const float s32 = (float)((double)amax / 448.0);
  if (ok) {
    uint32_t q = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) q |= f32_to_fp8_halfup(clip448(x[e] / s32)) << (8 * e);
    *reinterpret_cast<uint32_t*>(out + r * dim + c) = q;
  }
  if (l == 0) scales[r] = (uint8_t)f32_to_fp8_halfup(s32);
}

template <int TPR>
__global__ __launch_bounds__(256) void kv_dequant_fp8_vec_kernel(const uint8_t* __restrict__ codes,
                                                                 const uint8_t* __restrict__ scales,
                                                                 float* __restrict__ out, int64_t rows, int64_t dim) {
  const int64_t r = (int64_t)blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
  const int c = 4 * (threadIdx.x % TPR);
  if (r >= rows || c >= dim) return;
  const float sc = fp8_e4m3_to_f32(scales[r]);
  const uint32_t q = *reinterpret_cast<const uint32_t*>(codes + r * dim + c);
  f32x4 y;
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = sc > 0.f ? fp8_e4m3_to_f32((q >> (8 * e)) & 0xffu) * sc : 0.f;
  *reinterpret_cast<f32x4*>(out + r * dim + c) = y;
}

// threads per KV row for the vector kernels (0: the general kernels)
static int kv_tpr(int64_t dim, const void* a, const void* b) {
  if (dim % 4 != 0 || dim > 256 || !aligned(a, 16) || !aligned(b, 4)) return 0;
  int t = 1;
  while (4 * t < dim) t <<= 1;
  return t;
}

}  // namespace ccq

using namespace ccq;

extern "C" int ccq_quantize_rows_fp8(const uint16_t* w_bf16, const float* scale, uint8_t* out, int64_t rows,
                                     int64_t cols, void* stream) {
  CCQ_REQUIRE(rows >= 0 && cols >= 0, "ccq_quantize_rows_fp8: negative shape");
  CCQ_REQUIRE(rows <= 0x7fffffff, "ccq_quantize_rows_fp8: rows=%lld too large", (long long)rows);
  if (rows == 0 || cols == 0) return 0;
  CCQ_REQUIRE(w_bf16 && out, "ccq_quantize_rows_fp8: null pointer");
  hipStream_t st = as_stream(stream);
  const int64_t nv = cols / 8;
  if (cols % 8 == 0 && nv <= 2048 && aligned(w_bf16, 16) && aligned(out, 8)) {
    const dim3 g((unsigned)rows), b(256);
    if (nv <= 256)
      launch(quant_rows_fp8_vec_kernel<1>, g, b, 0, st, w_bf16, scale, out, cols);
    else if (nv <= 512)
      launch(quant_rows_fp8_vec_kernel<2>, g, b, 0, st, w_bf16, scale, out, cols);
    else if (nv <= 1024)
      launch(quant_rows_fp8_vec_kernel<4>, g, b, 0, st, w_bf16, scale, out, cols);
    else
      launch(quant_rows_fp8_vec_kernel<8>, g, b, 0, st, w_bf16, scale, out, cols);
  } else {
    launch(quant_rows_fp8_kernel, dim3((unsigned)rows), dim3(256), 0, st, w_bf16, scale, out, cols);
  }
  return launch_status("ccq_quantize_rows_fp8");
}

extern "C" int ccq_kv_quant_fp8(const float* kv, uint8_t* out, uint8_t* scales, int64_t rows, int64_t dim,
                                void* stream) {
  CCQ_REQUIRE(rows >= 0 && dim >= 0, "ccq_kv_quant_fp8: negative shape");
  CCQ_REQUIRE(rows <= 0x7fffffff, "ccq_kv_quant_fp8: rows=%lld too large", (long long)rows);
  if (rows == 0) return 0;
  CCQ_REQUIRE(kv && out && scales, "ccq_kv_quant_fp8: null pointer");
  hipStream_t st = as_stream(stream);
  const int tpr = kv_tpr(dim, kv, out);
#define CCQ_KVQ(T)                                                                                            \
  launch(kv_quant_fp8_vec_kernel<T>, dim3((unsigned)cdiv(rows, 256 / T)), dim3(256), 0, st, kv, out, \
                     scales, rows, dim)
  switch (tpr) {
    case 1: CCQ_KVQ(1); break;
    case 2: CCQ_KVQ(2); break;
    case 4: CCQ_KVQ(4); break;
    case 8: CCQ_KVQ(8); break;
    case 16: CCQ_KVQ(16); break;
    case 32: CCQ_KVQ(32); break;
    case 64: CCQ_KVQ(64); break;
    default: launch(kv_quant_fp8_kernel, dim3((unsigned)rows), dim3(256), 0, st, kv, out, scales, dim);
  }
#undef CCQ_KVQ
  return launch_status("ccq_kv_quant_fp8");
}

extern "C" int ccq_kv_dequant_fp8(const uint8_t* codes, const uint8_t* scales, float* out, int64_t rows,
                                  int64_t dim, void* stream) {
  CCQ_REQUIRE(rows >= 0 && dim >= 0, "ccq_kv_dequant_fp8: negative shape");
  CCQ_REQUIRE(rows <= 0x7fffffff, "ccq_kv_dequant_fp8: rows=%lld too large", (long long)rows);
  if (rows == 0 || dim == 0) return 0;
  CCQ_REQUIRE(codes && scales && out, "ccq_kv_dequant_fp8: null pointer");
  const int64_t n = rows * dim;
  hipStream_t st = as_stream(stream);
  const int tpr = kv_tpr(dim, out, codes);
#define CCQ_KVD(T)                                                                                          \
  launch(kv_dequant_fp8_vec_kernel<T>, dim3((unsigned)cdiv(rows, 256 / T)), dim3(256), 0, st, codes, \
                     scales, out, rows, dim)
  switch (tpr) {
    case 1: CCQ_KVD(1); break;
    case 2: CCQ_KVD(2); break;
    case 4: CCQ_KVD(4); break;
    case 8: CCQ_KVD(8); break;
    case 16: CCQ_KVD(16); break;
    case 32: CCQ_KVD(32); break;
    case 64: CCQ_KVD(64); break;
    default:
      launch(kv_dequant_fp8_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, codes, scales, out, n, dim);
  }
#undef CCQ_KVD
  return launch_status("ccq_kv_dequant_fp8");
}

extern "C" int ccq_fp8_to_f32(const uint8_t* code, float* out, int64_t n, void* stream) {
  CCQ_REQUIRE(n >= 0, "ccq_fp8_to_f32: n < 0");
  if (n == 0) return 0;
  CCQ_REQUIRE(code && out, "ccq_fp8_to_f32: null pointer");
  launch(fp8_to_f32_kernel, dim3(grid_for(n, 256)), dim3(256), 0, as_stream(stream), code, out, n);
  return launch_status("ccq_fp8_to_f32");
}

extern "C" int ccq_f32_to_fp8(const float* x, uint8_t* out, int64_t n, void* stream) {
  CCQ_REQUIRE(n >= 0, "ccq_f32_to_fp8: n < 0");
  if (n == 0) return 0;
  CCQ_REQUIRE(x && out, "ccq_f32_to_fp8: null pointer");
  launch(f32_to_fp8_kernel, dim3(grid_for(n, 256)), dim3(256), 0, as_stream(stream), x, out, n);
  return launch_status("ccq_f32_to_fp8");
}

extern "C" int ccq_group_broadcast_scale(const float* scale_groups, int64_t groups, int64_t group_size, float* out,
                                         void* stream) {
  CCQ_REQUIRE(groups >= 0 && group_size >= 0, "ccq_group_broadcast_scale: negative size");
  CCQ_REQUIRE(group_size == 0 || groups <= INT64_MAX / group_size, "ccq_group_broadcast_scale: size overflows");
  const int64_t n = groups * group_size;
  if (n == 0) return 0;
  CCQ_REQUIRE(scale_groups && out, "ccq_group_broadcast_scale: null pointer");
  launch(group_broadcast_kernel, dim3(grid_for(n, 256)), dim3(256), 0, as_stream(stream), scale_groups,
                     out, n, group_size);
  return launch_status("ccq_group_broadcast_scale");
}

extern "C" int ccq_silu_mul(const float* gate, const float* up, float* out, int64_t n, void* stream) {
  CCQ_REQUIRE(n >= 0, "ccq_silu_mul: n < 0");
  if (n == 0) return 0;
  CCQ_REQUIRE(gate && up && out, "ccq_silu_mul: null pointer");
  launch(silu_mul_kernel, dim3(grid_for(n, 256)), dim3(256), 0, as_stream(stream), gate, up, out, n);
  return launch_status("ccq_silu_mul");
}

extern "C" int ccq_fp8_dequant(const uint8_t* w, const float* scale, float* out, int64_t rows, int64_t cols,
                               void* stream) {
  CCQ_REQUIRE(rows >= 0 && cols >= 0, "ccq_fp8_dequant: negative shape");
  if (rows == 0 || cols == 0) return 0;
  CCQ_REQUIRE(w && scale && out, "ccq_fp8_dequant: null pointer");
  launch(fp8_dequant_kernel, dim3(grid_for(rows * cols, 256)), dim3(256), 0, as_stream(stream), w,
                     scale, out, rows, cols);
  return launch_status("ccq_fp8_dequant");
}

extern "C" int ccq_int4_dequant(const uint8_t* packed, const float* scale, float* out, int64_t rows,
                                int64_t cols, void* stream) {
  CCQ_REQUIRE(rows >= 0 && cols >= 0, "ccq_int4_dequant: negative shape");
  CCQ_REQUIRE(cols % 2 == 0, "ccq_int4_dequant: cols=%lld must be even (2 nibbles per byte)", (long long)cols);
  if (rows == 0 || cols == 0) return 0;
  CCQ_REQUIRE(packed && scale && out, "ccq_int4_dequant: null pointer");
  launch(int4_dequant_kernel, dim3(grid_for(rows * cols / 2, 256)), dim3(256), 0, as_stream(stream),
                     packed, scale, out, rows, cols);
  return launch_status("ccq_int4_dequant");
}

// Batch sizes from which the fp8 / int8 row-scale linears run on the MFMA
// kernel instead of the streaming one (measured at K=4096 N=14336: fp8
// 18.2 vs 20.4 us at 2 rows, the streaming kernel faster at 1; int8 18.2
// vs 26.1 us at 4 rows, the streaming kernel faster below).
constexpr int64_t kWqMinBatchFp8 = 2;
constexpr int64_t kWqMinBatchInt8 = 4;

static int ref_linear(int fmt, const float* x, const uint8_t* w, const float* scale, float* y, int64_t batch,
                      int64_t in_f, int64_t out_f, void* stream, const char* name, const float* table = nullptr,
                      int table_len = 0) {
  CCQ_REQUIRE(batch >= 0 && in_f >= 0 && out_f >= 0, "%s: negative shape", name);
  CCQ_REQUIRE((fmt != 0 && fmt != 3) || in_f % 2 == 0, "%s: in_features=%lld must be even", name, (long long)in_f);
  if (batch == 0 || out_f == 0) return 0;
  CCQ_REQUIRE(x && w && scale && y, "%s: null pointer", name);
  CCQ_REQUIRE(batch <= (int64_t)65535 * kLinBB, "%s: batch too large", name);
  dim3 grid((unsigned)cdiv(out_f, 4), (unsigned)cdiv(batch, kLinBB));
  CCQ_REQUIRE(grid.x <= 0x7fffffffu, "%s: out_features too large", name);
  if (in_f == 0) {  // empty sum; a fill kernel rather than a memset node
    launch(zero_f32_kernel, dim3(grid_for(batch * out_f, 256)), dim3(256), 0, as_stream(stream), y,
                       batch * out_f);
    return launch_status(name);
  }
  // fp8 / int8 batches from kWqMinBatch* rows: the decoded-weight MFMA
  // kernel, which reads W once per 64 rows (-1: shape it does not take)
  if ((fmt == 1 && batch >= kWqMinBatchFp8) || (fmt == 2 && batch >= kWqMinBatchInt8)) {
    const int rc = wq_mfma_linear(fmt == 1 ? WQ_FP8_ROW : WQ_INT8_ROW, x, w, scale, 0, 1.f, y, batch, in_f, out_f,
                                  as_stream(stream), name);
    if (rc >= 0) return rc;
  }
  // the streaming kernel: fp8 / int8 / int4 rows of whole 16-byte pieces,
  // 16-byte aligned, x rows that fit the staging area
  const int64_t rbytes = fmt == 0 ? in_f / 2 : in_f;
  if (fmt != 3 && rbytes % 16 == 0 && aligned(w, 16) && aligned(x, 16) && (fmt != 0 || aligned(scale, 16)) &&
      in_f * 4 <= RV_LDS) {
    // batch rows per pass: as many as the batch and the staging area allow
    int bb = 1;
    while (bb < 8 && bb * 2 <= batch && in_f * 4 * bb * 2 <= RV_LDS) bb *= 2;
    const dim3 g((unsigned)cdiv(out_f, 4 * (bb == 1 ? rv_rows<1>() : rv_rows<2>())), (unsigned)cdiv(batch, bb));
    CCQ_REQUIRE(cdiv(batch, bb) <= 65535, "%s: batch too large", name);
    const size_t lds = (size_t)bb * in_f * 4;
#define CCQ_RV(F, B) launch((ref_linear_vec_kernel<F, B>), g, dim3(256), lds, as_stream(stream), x, w, scale, y, batch, in_f, out_f)
#define CCQ_RV_B(F)   \
  do {                \
    if (bb == 8)      \
      CCQ_RV(F, 8);   \
    else if (bb == 4) \
      CCQ_RV(F, 4);   \
    else if (bb == 2) \
      CCQ_RV(F, 2);   \
    else              \
      CCQ_RV(F, 1);   \
  } while (0)
    if (fmt == 1)
      CCQ_RV_B(1);
    else if (fmt == 2)
      CCQ_RV_B(2);
    else
      CCQ_RV_B(0);
#undef CCQ_RV_B
#undef CCQ_RV
    return launch_status(name);
  }
  if (fmt == 1)
    launch(ref_linear_f32_kernel<1>, grid, dim3(256), 0, as_stream(stream), x, w, scale, y, batch,
                       in_f, out_f, table, table_len);
  else if (fmt == 2)
    launch(ref_linear_f32_kernel<2>, grid, dim3(256), 0, as_stream(stream), x, w, scale, y, batch,
                       in_f, out_f, table, table_len);
  else if (fmt == 3)
    launch(ref_linear_f32_kernel<3>, grid, dim3(256), 0, as_stream(stream), x, w, scale, y, batch,
                       in_f, out_f, table, table_len);
  else
    launch(ref_linear_f32_kernel<0>, grid, dim3(256), 0, as_stream(stream), x, w, scale, y, batch,
                       in_f, out_f, table, table_len);
  return launch_status(name);
}

extern "C" int ccq_int4_linear_f32(const float* x, const uint8_t* packed, const float* scale, float* y,
                                   int64_t batch, int64_t in_features, int64_t out_features, void* stream) {
  return ref_linear(0, x, packed, scale, y, batch, in_features, out_features, stream, "ccq_int4_linear_f32");
}

extern "C" int ccq_fp8_linear_f32(const float* x, const uint8_t* w, const float* scale, float* y, int64_t batch,
                                  int64_t in_features, int64_t out_features, void* stream) {
  return ref_linear(1, x, w, scale, y, batch, in_features, out_features, stream, "ccq_fp8_linear_f32");
}

extern "C" int ccq_nf4_linear_f32(const float* x, const uint8_t* packed, const float* scale, const float* table,
                                  int table_len, float* y, int64_t batch, int64_t in_features, int64_t out_features,
                                  void* stream) {
  CCQ_REQUIRE(table_len >= 0 && table_len <= 16, "ccq_nf4_linear_f32: table_len=%d outside [0, 16]", table_len);
  CCQ_REQUIRE(table || table_len == 0, "ccq_nf4_linear_f32: null table");
  return ref_linear(3, x, packed, scale, y, batch, in_features, out_features, stream, "ccq_nf4_linear_f32", table,
                    table_len);
}

extern "C" int ccq_nf4_dequant(const uint8_t* packed, const float* scale, const float* table, int table_len,
                               float* out, int64_t rows, int64_t cols, void* stream) {
  CCQ_REQUIRE(rows >= 0 && cols >= 0, "ccq_nf4_dequant: negative shape");
  CCQ_REQUIRE(cols % 2 == 0, "ccq_nf4_dequant: cols=%lld must be even (2 nibbles per byte)", (long long)cols);
  CCQ_REQUIRE(table_len >= 0 && table_len <= 16, "ccq_nf4_dequant: table_len=%d outside [0, 16]", table_len);
  if (rows == 0 || cols == 0) return 0;
  CCQ_REQUIRE(packed && scale && out && (table || table_len == 0), "ccq_nf4_dequant: null pointer");
  launch(nf4_dequant_kernel, dim3(grid_for(rows * cols / 2, 256)), dim3(256), 0, as_stream(stream),
                     packed, scale, table, table_len, out, rows, cols);
  return launch_status("ccq_nf4_dequant");
}

extern "C" int ccq_int8_quantize_cols(const float* x, const float* amax, int8_t* out, int64_t rows, int64_t cols,
                                      void* stream) {
  CCQ_REQUIRE(rows >= 0 && cols >= 0, "ccq_int8_quantize_cols: negative shape");
  if (rows == 0 || cols == 0) return 0;
  CCQ_REQUIRE(x && amax && out, "ccq_int8_quantize_cols: null pointer");
  launch(int8_quantize_cols_kernel, dim3(grid_for(rows * cols, 256)), dim3(256), 0, as_stream(stream),
                     x, amax, out, rows, cols);
  return launch_status("ccq_int8_quantize_cols");
}

extern "C" int ccq_int8_linear_f32(const float* x, const int8_t* w, const float* scale, float* y, int64_t batch,
                                   int64_t in_features, int64_t out_features, void* stream) {
  return ref_linear(2, x, reinterpret_cast<const uint8_t*>(w), scale, y, batch, in_features, out_features, stream,
                    "ccq_int8_linear_f32");
}
