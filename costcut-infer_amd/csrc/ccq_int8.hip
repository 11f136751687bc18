// INT8 linear of quant/int8.py:20-100: weights int8 [N, K] with one float32
// scale per output channel; W8A8 quantizes the activations per token
// (amax / 127, round half to even, clamp +-127, NaN -> 0), accumulates the int8
// products exactly in int32 and returns y = float32(acc) * x_scale * w_scale
// (two float32 roundings, in that order); W8A16 dequantizes the weight
// (w * scale, one rounding) for a float32 matmul.
//
// GEMM: v_mfma_i32_32x32x32_i8, a workgroup of 4 waves per 64 x 64 output
// tile (each wave 32 x 32), K in chunks of 64 staged in LDS.  Small M
// splits K over workgroups: each split writes its int32 partial tile to the
// workspace and a second kernel adds the splits (integer sums: any order
// gives the same result) and applies the float epilogue; with one split the
// GEMM applies it itself.
#include "ccq_common.h"

#include <math.h>

namespace ccq {

typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4v __attribute__((ext_vector_type(4)));

// Per token: amax = max|x| (NaN if the row holds one), amax' = amax if
// amax > 0 else 1, x_scale = amax' / 127 and factor = 127 / x_scale (float32
// divisions), q = clamp(rint(x * factor), -127, 127).
__global__ __launch_bounds__(256) void int8_act_quant_kernel(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                             float* __restrict__ xs, int64_t K) {
  __shared__ float red[4];
  __shared__ int rnan[4];
  const int64_t r = blockIdx.x;
  const float* row = x + r * K;
  float m = 0.f;
  int nan = 0;
  for (int64_t c = threadIdx.x; c < K; c += blockDim.x) {
    const float v = row[c];
    m = fmaxf(m, fabsf(v));
    nan |= v != v;
  }
  for (int off = 32; off >= 1; off >>= 1) {
    m = fmaxf(m, __shfl_xor(m, off, 64));
    nan |= __shfl_xor(nan, off, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    red[threadIdx.x >> 6] = m;
    rnan[threadIdx.x >> 6] = nan;
  }
  __syncthreads();
  const float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const bool anynan = (rnan[0] | rnan[1] | rnan[2] | rnan[3]) != 0;
  const float a = (!anynan && amax > 0.f) ? amax : 1.0f;
  const float scale = a / 127.0f;
  const float factor = 127.0f / scale;
  if (threadIdx.x == 0) xs[r] = scale;
  for (int64_t c = threadIdx.x; c < K; c += blockDim.x) {
    // numpy's float -> int8 cast turns NaN into 0 (observed on x86: the
    // truncating convert yields 0x80000000, whose low byte is 0)
    const float q = rintf(row[c] * factor);
    xq[r * K + c] = q != q ? (int8_t)0 : (int8_t)(int)fminf(fmaxf(q, -127.0f), 127.0f);
  }
}

constexpr int I8_BT = 64;         // output tile
constexpr int I8_KC = 64;         // K per LDS chunk
constexpr int I8_LDS_STRIDE = 80; // bytes per staged row (64 + 16: 16-byte aligned, fewer bank conflicts)

// acc of one 64 x 64 tile over k in [kb, ke) (multiples of 16, K % 16 == 0);
// the wave's 32 x 32 part in MFMA layout (register i: row 8*(i/4) + 4*h +
// i%4, column l%32, h = l/32)
__device__ __forceinline__ i32x16 int8_tile_acc(const int8_t* __restrict__ xq, const int8_t* __restrict__ w, int M,
                                               int N, int64_t K, int m0, int n0, int64_t kb, int64_t ke,
                                               int8_t (*As)[I8_LDS_STRIDE], int8_t (*Bs)[I8_LDS_STRIDE]) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave >> 1, wn = wave & 1;
  const int r = lane & 31, h = lane >> 5;
  const int lrow = t >> 2, seg = t & 3;  // staging: 64 rows x 4 segments of 16 B
  i32x16 acc = i32x16{};
  for (int64_t k0 = kb; k0 < ke; k0 += I8_KC) {
    const int64_t kk = k0 + 16 * seg;
    i32x4v av = i32x4v{}, bv = i32x4v{};
    if (m0 + lrow < M && kk < ke) av = *reinterpret_cast<const i32x4v*>(xq + (int64_t)(m0 + lrow) * K + kk);
    if (n0 + lrow < N && kk < ke) bv = *reinterpret_cast<const i32x4v*>(w + (int64_t)(n0 + lrow) * K + kk);
    __syncthreads();  // the previous chunk's reads are done
    *reinterpret_cast<i32x4v*>(&As[lrow][16 * seg]) = av;
    *reinterpret_cast<i32x4v*>(&Bs[lrow][16 * seg]) = bv;
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const i32x4v a = *reinterpret_cast<const i32x4v*>(&As[wm * 32 + r][32 * s + 16 * h]);
      const i32x4v b = *reinterpret_cast<const i32x4v*>(&Bs[wn * 32 + r][32 * s + 16 * h]);
      acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc, 0, 0, 0);
    }
  }
  return acc;
}

// one split of K per blockIdx.z; splits == 1: the float epilogue here,
// else int32 partials to part[z][M][N]
__global__ __launch_bounds__(256) void int8_gemm_kernel(const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                        const int8_t* __restrict__ w, const float* __restrict__ ws,
                                                        float* __restrict__ y, int32_t* __restrict__ part, int M,
                                                        int N, int64_t K, int64_t kper) {
  __shared__ __align__(16) int8_t As[I8_BT][I8_LDS_STRIDE];
  __shared__ __align__(16) int8_t Bs[I8_BT][I8_LDS_STRIDE];
  const int n0 = blockIdx.x * I8_BT, m0 = blockIdx.y * I8_BT;
  const int64_t kb = (int64_t)blockIdx.z * kper, ke = kb + kper < K ? kb + kper : K;
  const i32x16 acc = int8_tile_acc(xq, w, M, N, K, m0, n0, kb, ke, As, Bs);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wm = wave >> 1, wn = wave & 1;
  const int col = n0 + wn * 32 + (lane & 31), h = lane >> 5;
  if (col >= N) return;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = m0 + wm * 32 + 8 * (i / 4) + 4 * h + (i % 4);
    if (row >= M) continue;
    if (gridDim.z == 1)
      y[(int64_t)row * N + col] = ((float)acc[i] * xs[row]) * ws[col];
    else
      part[((int64_t)blockIdx.z * M + row) * N + col] = acc[i];
  }
}

__global__ void int8_splitk_epilogue_kernel(const int32_t* __restrict__ part, const float* __restrict__ xs,
                                            const float* __restrict__ ws, float* __restrict__ y, int M, int N,
                                            int splits) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)M * N) return;
  const int row = (int)(i / N), col = (int)(i - (int64_t)row * N);
  int32_t acc = 0;
  for (int z = 0; z < splits; ++z) acc += part[(int64_t)z * M * N + i];
  y[i] = ((float)acc * xs[row]) * ws[col];
}

// K not a multiple of 16 (or 0): one thread per output, exact int32 sum
__global__ void int8_gemm_scalar_kernel(const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                        const int8_t* __restrict__ w, const float* __restrict__ ws,
                                        float* __restrict__ y, int M, int N, int64_t K) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)M * N) return;
  const int row = (int)(i / N), col = (int)(i - (int64_t)row * N);
  int32_t acc = 0;
  for (int64_t k = 0; k < K; ++k) acc += (int32_t)xq[(int64_t)row * K + k] * (int32_t)w[(int64_t)col * K + k];
  y[i] = ((float)acc * xs[row]) * ws[col];
}

// out[r, c] = w[r, c] * scale[r] (an 8-bit integer times a float32: one rounding)
__global__ void int8_dequant_kernel(const int8_t* __restrict__ w, const float* __restrict__ scale,
                                    float* __restrict__ out, int64_t rows, int64_t cols) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < rows * cols; i += stride) out[i] = (float)w[i] * scale[i / cols];
}

// K splits for an M x N problem: enough workgroups to cover the compute
// units about twice, each split at least 512 deep
int int8_splits(int64_t M, int64_t K, int64_t N) {
  if (K % 16 != 0) return 1;
  const int64_t tiles = cdiv(M, I8_BT) * cdiv(N, I8_BT);
  int64_t s = 1;
  while (tiles * s < 512 && K / (2 * s) >= 512 && s < 64) s *= 2;
  return (int)s;
}

}  // namespace ccq

using namespace ccq;

extern "C" int ccq_int8_act_quant(const float* x, int8_t* xq, float* x_scale, int64_t M, int64_t K, void* stream) {
  CCQ_REQUIRE(M >= 0 && K >= 0, "ccq_int8_act_quant: negative shape");
  CCQ_REQUIRE(M <= 0x7fffffff, "ccq_int8_act_quant: M=%lld too large", (long long)M);
  if (M == 0) return 0;
  CCQ_REQUIRE(x && xq && x_scale, "ccq_int8_act_quant: null pointer");
  hipLaunchKernelGGL(int8_act_quant_kernel, dim3((unsigned)M), dim3(256), 0, as_stream(stream), x, xq, x_scale, K);
  return launch_status("ccq_int8_act_quant");
}

extern "C" size_t ccq_int8_linear_workspace_size(int64_t M, int64_t K, int64_t N) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  const int s = int8_splits(M, K, N);
  return s > 1 ? (size_t)s * (size_t)M * (size_t)N * 4 : 0;
}

extern "C" int ccq_int8_linear(const int8_t* xq, const float* x_scale, const int8_t* w, const float* w_scale,
                               float* y, int64_t M, int64_t K, int64_t N, void* workspace,
                               size_t workspace_bytes, void* stream) {
  CCQ_REQUIRE(M >= 0 && K >= 0 && N >= 0, "ccq_int8_linear: negative shape");
  CCQ_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff, "ccq_int8_linear: M or N too large");
  CCQ_REQUIRE(K < (1 << 17), "ccq_int8_linear: K=%lld >= 131072 could overflow the int32 sums", (long long)K);
  if (M == 0 || N == 0) return 0;
  CCQ_REQUIRE(xq && x_scale && w && w_scale && y, "ccq_int8_linear: null pointer");
  hipStream_t st = as_stream(stream);
  if (K == 0 || K % 16 != 0 || !aligned(xq, 16) || !aligned(w, 16)) {  // exact per-output sums
    const int64_t n = M * N;
    hipLaunchKernelGGL(int8_gemm_scalar_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st, xq, x_scale, w,
                       w_scale, y, (int)M, (int)N, K);
    return launch_status("ccq_int8_linear");
  }
  const int s = int8_splits(M, K, N);
  const size_t need = ccq_int8_linear_workspace_size(M, K, N);
  CCQ_REQUIRE(s == 1 || (workspace && workspace_bytes >= need && aligned(workspace, 16)),
              "ccq_int8_linear: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  CCQ_REQUIRE(cdiv(M, I8_BT) <= 65535, "ccq_int8_linear: M=%lld too large", (long long)M);
  const int64_t kper = cdiv(cdiv(K, s), I8_KC) * I8_KC;
  const dim3 grid((unsigned)cdiv(N, I8_BT), (unsigned)cdiv(M, I8_BT), (unsigned)cdiv(K, kper));
  hipLaunchKernelGGL(int8_gemm_kernel, grid, dim3(256), 0, st, xq, x_scale, w, w_scale, y, (int32_t*)workspace,
                     (int)M, (int)N, K, kper);
  if (grid.z > 1)
    hipLaunchKernelGGL(int8_splitk_epilogue_kernel, dim3((unsigned)cdiv(M * N, 256)), dim3(256), 0, st,
                       (const int32_t*)workspace, x_scale, w_scale, y, (int)M, (int)N, (int)grid.z);
  return launch_status("ccq_int8_linear");
}

extern "C" int ccq_int8_dequant(const int8_t* w, const float* scale, float* out, int64_t rows, int64_t cols,
                                void* stream) {
  CCQ_REQUIRE(rows >= 0 && cols >= 0, "ccq_int8_dequant: negative shape");
  if (rows == 0 || cols == 0) return 0;
  CCQ_REQUIRE(w && scale && out, "ccq_int8_dequant: null pointer");
  hipLaunchKernelGGL(int8_dequant_kernel, dim3(grid_for(rows * cols, 256)), dim3(256), 0, as_stream(stream), w,
                     scale, out, rows, cols);
  return launch_status("ccq_int8_dequant");
}
