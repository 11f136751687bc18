// MX formats of quant/mx.py:21-94 and kernels.py:240-256: weights [out, in]
// in groups of G consecutive input columns per output row, each group with
// one E8M0 scale byte e (scale = 2^(e-127); e = 0 -> 0, e = 255 -> NaN),
// scales laid out [out, ceil(in / G)].
//   fmt 0, MXFP8: one e4m3fn code per byte, W = fp8(code) * scale.
//   fmt 1, MXFP4 / NVFP4: two 4-bit codes per byte (low nibble = even
//   column), W = (lut[code] * scale) * scale2, with the reference's table
//   lut = {0, .5, 1, 1.5, -0, -.5, -1, -1.5} repeated for codes 8..15 (not
//   OCP E2M1), the scale optional and scale2 NVFP4's per-tensor factor
//   (1 leaves W unchanged).
// The layer is y = x @ W.T in float32 with W formed on the fly.
#include "ccq_common.h"

#include <math.h>

namespace ccq {

__device__ __forceinline__ float mx4_lut(uint32_t code) {
  const uint32_t m = code & 3u;  // 0, .5, 1, 1.5: exact as m * 0.5
  const float v = (float)m * 0.5f;
  return (code & 4u) ? -v : v;
}

template <bool kFp4>
__device__ __forceinline__ float mx_weight(const uint8_t* __restrict__ w, const uint8_t* __restrict__ sc,
                                           int64_t r, int64_t c, int64_t cols, int G, int64_t gpr, float s2) {
  float v;
  if (kFp4) {
    const uint32_t b = w[r * (cols / 2) + (c >> 1)];
    v = mx4_lut((c & 1) ? b >> 4 : b & 15u);
  } else {
    v = fp8_e4m3_to_f32(w[r * cols + c]);
  }
  if (sc) v = v * e8m0_to_f32(sc[r * gpr + c / G]);
  return kFp4 ? v * s2 : v;
}

__global__ void e8m0_to_f32_kernel(const uint8_t* __restrict__ e, float* __restrict__ out, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) out[i] = e8m0_to_f32(e[i]);
}

template <bool kFp4>
__global__ void mx_dequant_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ sc,
                                  float* __restrict__ out, int64_t rows, int64_t cols, int G, float s2) {
  const int64_t gpr = cdiv(cols, G);
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < rows * cols; i += stride) {
    const int64_t r = i / cols, c = i - r * cols;
    out[i] = mx_weight<kFp4>(w, sc, r, c, cols, G, gpr, s2);
  }
}

// a wave per output row, 8 batch rows per workgroup (blockIdx.y)
constexpr int kMxBB = 8;
// batch size from which the layer runs on the decoded-weight MFMA kernel
// (measured faster than the vector kernel from one row: K=4096 N=14336
// MXFP8 23.6 vs 30.4 us, MXFP4 22.1 vs 24.5 us)
constexpr int64_t kMxWqMinBatch = 1;

template <bool kFp4>
__global__ __launch_bounds__(256) void mx_linear_f32_kernel(const float* __restrict__ x, const uint8_t* __restrict__ w,
                                                            const uint8_t* __restrict__ sc, float* __restrict__ y,
                                                            int64_t batch, int64_t in_f, int64_t out_f, int G,
                                                            float s2) {
  const int lane = lane_id();
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= out_f) return;
  const int64_t b0 = (int64_t)blockIdx.y * kMxBB;
  const int nb = (int)min<int64_t>(kMxBB, batch - b0);
  const int64_t gpr = cdiv(in_f, G);
  float acc[kMxBB];
#pragma unroll
  for (int b = 0; b < kMxBB; ++b) acc[b] = 0.f;
  for (int64_t c = lane; c < in_f; c += 64) {
    const float wv = mx_weight<kFp4>(w, sc, r, c, in_f, G, gpr, s2);
#pragma unroll
    for (int b = 0; b < kMxBB; ++b)
      if (b < nb) acc[b] = fmaf(x[(b0 + b) * in_f + c], wv, acc[b]);
  }
#pragma unroll
  for (int b = 0; b < kMxBB; ++b) {
    float v = acc[b];
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    acc[b] = v;
  }
  if (lane == 0)
    for (int b = 0; b < nb; ++b) y[(b0 + b) * out_f + r] = acc[b];
}

// Vector form for in_features % 32 == 0, group_size 16 or 32, 16-byte
// aligned operands: a lane takes 16 weight bytes at a time (32 FP4 or 16
// FP8 columns, inside one or two scale groups), each wave 4 weight rows that
// share the activation loads, each workgroup 16 rows and up to 8 batch rows.
// Decode: FP4 through mx4_word (one v_perm_b32 per 4 codes); FP8 through the hardware
// e4m3fn converter (v_cvt_pk_f32_fp8).  The E8M0 scale (a power of two, 0
// or NaN) multiplies each group's partial sum once; NVFP4's second scale
// multiplies the row's sum.  This is not the reference's arithmetic, which
// forms W = (lut * s) * scale2 per weight and then multiplies: a
// power-of-two s rescales every term exactly only while products stay
// normal (near e8m0 1 the subnormal roundings differ; at e8m0 254 the
// reference's W can overflow to inf, and a zero activation times inf gives
// NaN where the kernel gives 0), and scale2 is an arbitrary float32, so
// applying it once to the sum rounds differently from applying it to each
// weight.  Both differences are within float32 summation-order tolerance
// for finite, normal-range scales.
constexpr int kMxRPW = 4;

template <bool kFp4, int G>
__global__ __launch_bounds__(256) void mx_linear_f32_vec_kernel(const float* __restrict__ x,
                                                                const uint8_t* __restrict__ w,
                                                                const uint8_t* __restrict__ sc,
                                                                float* __restrict__ y, int64_t batch, int64_t in_f,
                                                                int64_t out_f, float s2) {
  constexpr int VPU = kFp4 ? 32 : 16;          // columns per 16-byte unit
  constexpr int NG = (kFp4 && G == 16) ? 2 : 1;  // scale groups per unit
  constexpr int GPU_ = VPU / NG;                // columns per group inside the unit
  const int lane = lane_id();
  const int64_t r0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * kMxRPW;
  if (r0 >= out_f) return;
  const int64_t b0 = (int64_t)blockIdx.y * kMxBB;
  const int nb = (int)min<int64_t>(kMxBB, batch - b0);
  const int64_t units = in_f / VPU, row_bytes = kFp4 ? in_f / 2 : in_f, gpr = in_f / G;
  float acc[kMxBB][kMxRPW];
#pragma unroll
  for (int b = 0; b < kMxBB; ++b)
#pragma unroll
    for (int q = 0; q < kMxRPW; ++q) acc[b][q] = 0.f;
  for (int64_t u = lane; u < units; u += 64) {
    const int64_t c0 = u * VPU;
    uint4 wb[kMxRPW];
    float sg[kMxRPW][NG];
#pragma unroll
    for (int q = 0; q < kMxRPW; ++q) {
      const int64_t r = min<int64_t>(r0 + q, out_f - 1);
      wb[q] = *reinterpret_cast<const uint4*>(w + r * row_bytes + u * 16);
#pragma unroll
      for (int g = 0; g < NG; ++g) sg[q][g] = sc ? e8m0_to_f32(sc[r * gpr + (c0 + g * GPU_) / G]) : 1.f;
    }
    // activations once per unit and batch row, shared by the 4 weight rows
    // (the rows' codes are decoded per batch row: a few VALU per value)
#pragma unroll
    for (int b = 0; b < kMxBB; ++b) {
      if (b < nb) {
        const float4* xr = reinterpret_cast<const float4*>(x + (b0 + b) * in_f + c0);
        float xv[VPU];
#pragma unroll
        for (int j4 = 0; j4 < VPU / 4; ++j4) {
          const float4 v4 = xr[j4];
          xv[4 * j4] = v4.x;
          xv[4 * j4 + 1] = v4.y;
          xv[4 * j4 + 2] = v4.z;
          xv[4 * j4 + 3] = v4.w;
        }
#pragma unroll
        for (int q = 0; q < kMxRPW; ++q) {
          float wv[VPU];
          const uint32_t words[4] = {wb[q].x, wb[q].y, wb[q].z, wb[q].w};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            if constexpr (kFp4) {
              float v8[8];
              mx4_word(words[t], v8);
#pragma unroll
              for (int j = 0; j < 8; ++j) wv[8 * t + j] = v8[j];
            } else {
              const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)words[t], false);
              const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)words[t], true);
              wv[4 * t] = lo[0];
              wv[4 * t + 1] = lo[1];
              wv[4 * t + 2] = hi[0];
              wv[4 * t + 3] = hi[1];
            }
          }
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            float part = 0.f;
#pragma unroll
            for (int j = g * GPU_; j < (g + 1) * GPU_; ++j) part = fmaf(xv[j], wv[j], part);
            acc[b][q] = fmaf(part, sg[q][g], acc[b][q]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int b = 0; b < kMxBB; ++b)
#pragma unroll
    for (int q = 0; q < kMxRPW; ++q) {
      float v = acc[b][q];
      for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
      acc[b][q] = kFp4 ? v * s2 : v;
    }
  if (lane == 0)
    for (int b = 0; b < nb; ++b)
#pragma unroll
      for (int q = 0; q < kMxRPW; ++q)
        if (r0 + q < out_f) y[(b0 + b) * out_f + r0 + q] = acc[b][q];
}

// Dequant, vector form (cols % 32 == 0, G in {16, 32}, 16-byte aligned):
// one thread per 16 weight bytes, float4 stores.
template <bool kFp4, int G>
__global__ void mx_dequant_vec_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ sc,
                                      float* __restrict__ out, int64_t rows, int64_t cols, float s2) {
  constexpr int VPU = kFp4 ? 32 : 16;
  const int64_t upr = cols / VPU, gpr = cols / G;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < rows * upr; i += stride) {
    const int64_t r = i / upr, u = i - r * upr, c0 = u * VPU;
    const uint4 wb = *reinterpret_cast<const uint4*>(w + i * 16);
    const float sg0 = sc ? e8m0_to_f32(sc[r * gpr + c0 / G]) : 1.f;
    const float sg1 = sc ? e8m0_to_f32(sc[r * gpr + (c0 + VPU - 1) / G]) : 1.f;
    const uint32_t words[4] = {wb.x, wb.y, wb.z, wb.w};
    float4* o = reinterpret_cast<float4*>(out + r * cols + c0);
#pragma unroll
    for (int j4 = 0; j4 < VPU / 4; ++j4) {
      float v[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int j = 4 * j4 + t;
        const uint32_t word = words[kFp4 ? j / 8 : j / 4];
        float x = kFp4 ? mx4_lut((word >> (4 * (j % 8))) & 15u) : fp8_e4m3_to_f32((word >> (8 * (j % 4))) & 255u);
        if (sc) x = x * (j < G - (int)(c0 % G) ? sg0 : sg1);
        v[t] = kFp4 ? x * s2 : x;
      }
      o[j4] = make_float4(v[0], v[1], v[2], v[3]);
    }
  }
}

}  // namespace ccq

using namespace ccq;

static int mx_check(int fmt, int64_t rows, int64_t cols, int G, const uint8_t* sc, const char* name) {
  CCQ_REQUIRE(fmt == 0 || fmt == 1, "%s: fmt=%d (0 MXFP8, 1 MXFP4/NVFP4)", name, fmt);
  CCQ_REQUIRE(rows >= 0 && cols >= 0, "%s: negative shape", name);
  CCQ_REQUIRE(G > 0, "%s: group_size=%d must be positive", name, G);
  CCQ_REQUIRE(fmt == 1 || sc, "%s: MXFP8 needs its E8M0 scales", name);
  CCQ_REQUIRE(fmt == 0 || cols % 2 == 0, "%s: in_features=%lld must be even for 4-bit codes", name,
              (long long)cols);
  return 0;
}

extern "C" int ccq_e8m0_to_f32(const uint8_t* e8m0, float* out, int64_t n, void* stream) {
  CCQ_REQUIRE(n >= 0, "ccq_e8m0_to_f32: negative size");
  if (n == 0) return 0;
  CCQ_REQUIRE(e8m0 && out, "ccq_e8m0_to_f32: null pointer");
  launch(e8m0_to_f32_kernel, dim3(grid_for(n, 256)), dim3(256), 0, as_stream(stream), e8m0, out, n);
  return launch_status("ccq_e8m0_to_f32");
}

extern "C" int ccq_mx_dequant(const uint8_t* w, const uint8_t* scale_e8m0, float* out, int64_t rows, int64_t cols,
                              int fmt, int group_size, float scale2, void* stream) {
  if (int rc = mx_check(fmt, rows, cols, group_size, scale_e8m0, "ccq_mx_dequant")) return rc;
  if (rows == 0 || cols == 0) return 0;
  CCQ_REQUIRE(w && out, "ccq_mx_dequant: null pointer");
  if (cols % 32 == 0 && (group_size == 16 || group_size == 32) && aligned(w, 16) && aligned(out, 16)) {
    const int64_t units = rows * (cols / (fmt == 1 ? 32 : 16));
    const dim3 g(grid_for(units, 256));
    hipStream_t st = as_stream(stream);
    if (fmt == 1 && group_size == 32)
      launch((mx_dequant_vec_kernel<true, 32>), g, dim3(256), 0, st, w, scale_e8m0, out, rows, cols, scale2);
    else if (fmt == 1)
      launch((mx_dequant_vec_kernel<true, 16>), g, dim3(256), 0, st, w, scale_e8m0, out, rows, cols, scale2);
    else if (group_size == 32)
      launch((mx_dequant_vec_kernel<false, 32>), g, dim3(256), 0, st, w, scale_e8m0, out, rows, cols,
                         scale2);
    else
      launch((mx_dequant_vec_kernel<false, 16>), g, dim3(256), 0, st, w, scale_e8m0, out, rows, cols,
                         scale2);
    return launch_status("ccq_mx_dequant");
  }
  const dim3 grid(grid_for(rows * cols, 256));
  if (fmt == 1)
    launch(mx_dequant_kernel<true>, grid, dim3(256), 0, as_stream(stream), w, scale_e8m0, out, rows,
                       cols, group_size, scale2);
  else
    launch(mx_dequant_kernel<false>, grid, dim3(256), 0, as_stream(stream), w, scale_e8m0, out, rows,
                       cols, group_size, scale2);
  return launch_status("ccq_mx_dequant");
}

extern "C" int ccq_mx_linear_f32(const float* x, const uint8_t* w, const uint8_t* scale_e8m0, float* y,
                                 int64_t batch, int64_t in_features, int64_t out_features, int fmt, int group_size,
                                 float scale2, void* stream) {
  if (int rc = mx_check(fmt, out_features, in_features, group_size, scale_e8m0, "ccq_mx_linear_f32")) return rc;
  CCQ_REQUIRE(batch >= 0, "ccq_mx_linear_f32: negative batch");
  if (batch == 0 || out_features == 0) return 0;
  CCQ_REQUIRE(x && w && y, "ccq_mx_linear_f32: null pointer");
  if (batch >= kMxWqMinBatch) {  // the decoded-weight MFMA kernel (-1: a shape it does not take)
    const int rc = wq_mfma_linear(fmt == 0 ? WQ_MXFP8 : WQ_MXFP4, x, w, scale_e8m0, group_size, scale2, y, batch,
                                  in_features, out_features, as_stream(stream), "ccq_mx_linear_f32");
    if (rc >= 0) return rc;
  }
  CCQ_REQUIRE(cdiv(batch, kMxBB) <= 65535, "ccq_mx_linear_f32: batch too large");
  if (in_features % 32 == 0 && in_features > 0 && (group_size == 16 || group_size == 32) && aligned(x, 16) &&
      aligned(w, 16)) {
    const dim3 grid((unsigned)cdiv(out_features, 4 * kMxRPW), (unsigned)cdiv(batch, kMxBB));
    hipStream_t st = as_stream(stream);
    if (fmt == 1 && group_size == 32)
      launch((mx_linear_f32_vec_kernel<true, 32>), grid, dim3(256), 0, st, x, w, scale_e8m0, y, batch,
                         in_features, out_features, scale2);
    else if (fmt == 1)
      launch((mx_linear_f32_vec_kernel<true, 16>), grid, dim3(256), 0, st, x, w, scale_e8m0, y, batch,
                         in_features, out_features, scale2);
    else if (group_size == 32)
      launch((mx_linear_f32_vec_kernel<false, 32>), grid, dim3(256), 0, st, x, w, scale_e8m0, y, batch,
                         in_features, out_features, scale2);
    else
      launch((mx_linear_f32_vec_kernel<false, 16>), grid, dim3(256), 0, st, x, w, scale_e8m0, y, batch,
                         in_features, out_features, scale2);
    return launch_status("ccq_mx_linear_f32");
  }
  const dim3 grid((unsigned)cdiv(out_features, 4), (unsigned)cdiv(batch, kMxBB));
  if (fmt == 1)
    launch(mx_linear_f32_kernel<true>, grid, dim3(256), 0, as_stream(stream), x, w, scale_e8m0, y,
                       batch, in_features, out_features, group_size, scale2);
  else
    launch(mx_linear_f32_kernel<false>, grid, dim3(256), 0, as_stream(stream), x, w, scale_e8m0, y,
                       batch, in_features, out_features, group_size, scale2);
  return launch_status("ccq_mx_linear_f32");
}
