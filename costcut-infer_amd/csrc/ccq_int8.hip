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

// The same for rows of K <= 1024 * VPT floats (K % 4 == 0, 16-byte aligned
// rows): each thread loads its VPT float4 at once and keeps them in
// registers for the quantization, one round of loads per row.
template <int VPT>
__global__ __launch_bounds__(256) void int8_act_quant_vec_kernel(const float* __restrict__ x,
                                                                 int8_t* __restrict__ xq, float* __restrict__ xs,
                                                                 int64_t K) {
  __shared__ float red[4];
  __shared__ int rnan[4];
  const int64_t r = blockIdx.x;
  const float4* row = reinterpret_cast<const float4*>(x + r * K);
  const int n4 = (int)(K >> 2);
  float4 v[VPT];
  float m = 0.f;
  int nan = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = threadIdx.x + 256 * i;
    v[i] = c < n4 ? row[c] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    m = fmaxf(fmaxf(m, fmaxf(fabsf(v[i].x), fabsf(v[i].y))), fmaxf(fabsf(v[i].z), fabsf(v[i].w)));
    nan |= (v[i].x != v[i].x) | (v[i].y != v[i].y) | (v[i].z != v[i].z) | (v[i].w != v[i].w);
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
  auto q8 = [&](float f) -> uint32_t {
    const float q = rintf(f * factor);
    return q != q ? 0u : (uint32_t)(uint8_t)(int8_t)(int)fminf(fmaxf(q, -127.0f), 127.0f);
  };
  uint32_t* out = reinterpret_cast<uint32_t*>(xq + r * K);
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = threadIdx.x + 256 * i;
    if (c < n4) out[c] = q8(v[i].x) | (q8(v[i].y) << 8) | (q8(v[i].z) << 16) | (q8(v[i].w) << 24);
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

// Skinny GEMM for M <= 32 (decode): a workgroup owns 32 output columns and a
// K range; its 4 waves take the range's 128-deep chunks in turn (adjacent
// chunks of the same weight rows at once).  A chunk (32 rows x 128 B) is
// read as 4 loads of 8 whole rows' 128 B each (lane l: row 8p + l/8, bytes
// 16*(l%8)), SK_D chunks ahead of the MFMAs, and turned into MFMA layout
// through the wave's own LDS tile.  MFMA step p uses bytes [16p, 16p+16)
// of lane half h's 64-byte run, so lane half h covers k = k0 + 64h + 16p +
// j in both operands: a fixed permutation of k, which leaves the integer
// sums exact.  The activations (rows l%32 < M, L2-resident) are read in
// MFMA layout directly.
constexpr int SK_D = 4;          // chunks in flight per wave
constexpr int SK_TROW = 144;     // bytes per LDS tile row (128 + 16)

// kFused (M <= I8_FUSED_M): the activations come as float32; every
// workgroup takes each row's amax over all of K (the rows are L2-resident;
// the weight prefetch is already in flight), quantizes its own K range into
// LDS exactly as int8_act_quant_vec_kernel does, and workgroup (0, 0)
// stores the row scales to xs_out.  Otherwise xq / xs are the quantized
// activations and their scales.
constexpr int I8_FUSED_M = 4;
constexpr int I8_FUSED_XA = 16384;  // LDS bytes for the quantized K range of all rows

template <bool kFused>
__global__ __launch_bounds__(256) void int8_gemm_skinny_kernel(const int8_t* __restrict__ xq,
                                                               const float* __restrict__ xf,
                                                               float* __restrict__ xs_out,
                                                               const float* __restrict__ xs,
                                                               const int8_t* __restrict__ w,
                                                               const float* __restrict__ ws, float* __restrict__ y,
                                                               int32_t* __restrict__ part, int M, int N, int64_t K,
                                                               int64_t kper) {
  __shared__ __align__(16) int8_t tile[4][32 * SK_TROW];
  __shared__ int32_t red[4][16][64];
  __shared__ __align__(16) int8_t xa[kFused ? I8_FUSED_XA : 16];
  __shared__ float xsl[I8_FUSED_M], pmax[4][I8_FUSED_M];
  __shared__ int pnan[4][I8_FUSED_M];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 31, h = lane >> 5;
  const int n0 = blockIdx.x * 32;
  const int64_t kb = (int64_t)blockIdx.y * kper, ke = kb + kper < K ? kb + kper : K;
  const int nchunks = (int)cdiv(ke - kb, 128);
  const int mine = nchunks > wave ? (nchunks - wave + 3) / 4 : 0;  // chunks wave, wave+4, ...
  // Buffer loads: an offset at or past the buffer's size reads zeros without
  // touching memory, which zeroes rows past N or M and k past the range
  // with no branch around the loads (N*K and M*K < 2^31, checked by the host).
  constexpr uint32_t kOut = 0x80000000u;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, (int)(N * K), 0x00020000);
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc((void*)(kFused ? nullptr : xq), (short)0, kFused ? 0 : (int)(M * K), 0x00020000);
  const int lr = lane >> 3, lc = 16 * (lane & 7);  // load layout: row lr (+8p), byte lc of the chunk
  uint32_t wrow[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) wrow[p] = n0 + 8 * p + lr < N ? (uint32_t)((n0 + 8 * p + lr) * K) : kOut;
  const uint32_t xrow = r < M ? (uint32_t)(r * K) : kOut;
  int8_t* tw = tile[wave];
  i32x4v bq[SK_D][4], aq[kFused ? 1 : SK_D][4];
  auto load = [&](int c, i32x4v (&b)[4], i32x4v (&a)[4]) {
    const uint32_t k0 = (uint32_t)(kb + (int64_t)(wave + 4 * c) * 128);
    const bool okb = k0 + lc < (uint32_t)ke;  // ke is a multiple of 16
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      b[p] = __builtin_amdgcn_raw_buffer_load_b128(wr, okb ? wrow[p] + k0 + lc : kOut, 0, 0);
      if (!kFused) {
        const uint32_t ka = k0 + 64 * h + 16 * p;
        a[p] = __builtin_amdgcn_raw_buffer_load_b128(xr, ka < (uint32_t)ke ? xrow + ka : kOut, 0, 0);
      }
    }
  };
  // Chunks past the wave's last one lie at k >= ke and load as zeros, so the
  // prefetch and the MFMAs run unconditionally (a branch-free loop lets the
  // compiler wait only for the oldest slot's loads).
#pragma unroll
  for (int d = 0; d < SK_D; ++d) load(d, bq[d], aq[kFused ? 0 : d]);
  const int kstride = (int)kper;  // bytes per row of xa
  if constexpr (kFused) {
    // row amax over all of K (NaN flagged apart, as numpy's max propagates it)
    for (int m = 0; m < M; ++m) {
      const float4* xr4 = reinterpret_cast<const float4*>(xf + (int64_t)m * K);
      float mx = 0.f;
      int nan = 0;
#pragma unroll 4
      for (int c = threadIdx.x; c < (int)(K >> 2); c += 256) {
        const float4 v = xr4[c];
        mx = fmaxf(fmaxf(mx, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
        nan |= (v.x != v.x) | (v.y != v.y) | (v.z != v.z) | (v.w != v.w);
      }
      for (int off = 32; off >= 1; off >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        nan |= __shfl_xor(nan, off, 64);
      }
      if (lane == 0) {
        pmax[wave][m] = mx;
        pnan[wave][m] = nan;
      }
    }
    __syncthreads();
    if (threadIdx.x < M) {
      const int m = threadIdx.x;
      const float amax = fmaxf(fmaxf(pmax[0][m], pmax[1][m]), fmaxf(pmax[2][m], pmax[3][m]));
      const bool anynan = (pnan[0][m] | pnan[1][m] | pnan[2][m] | pnan[3][m]) != 0;
      const float a = (!anynan && amax > 0.f) ? amax : 1.0f;
      const float scale = a / 127.0f;
      xsl[m] = scale;
      if (blockIdx.x == 0 && blockIdx.y == 0) xs_out[m] = scale;
    }
    __syncthreads();
    // this workgroup's K range of every row, quantized into xa[m][k - kb]
    const int kr4 = (int)((ke - kb) >> 2);
    for (int m = 0; m < M; ++m) {
      const float factor = 127.0f / xsl[m];
      const float4* xr4 = reinterpret_cast<const float4*>(xf + (int64_t)m * K + kb);
      uint32_t* xo = reinterpret_cast<uint32_t*>(xa + m * kstride);
      auto q8 = [&](float f) -> uint32_t {
        const float q = rintf(f * factor);
        return q != q ? 0u : (uint32_t)(uint8_t)(int8_t)(int)fminf(fmaxf(q, -127.0f), 127.0f);
      };
      for (int c = threadIdx.x; c < kr4; c += 256) {
        const float4 v = xr4[c];
        xo[c] = q8(v.x) | (q8(v.y) << 8) | (q8(v.z) << 16) | (q8(v.w) << 24);
      }
    }
    __syncthreads();
  }
  i32x16 acc = i32x16{};
  for (int c0 = 0; c0 < mine; c0 += SK_D) {
#pragma unroll
    for (int d = 0; d < SK_D; ++d) {
#pragma unroll
      for (int p = 0; p < 4; ++p) *reinterpret_cast<i32x4v*>(tw + (8 * p + lr) * SK_TROW + lc) = bq[d][p];
      i32x4v bm[4], am[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) bm[p] = *reinterpret_cast<const i32x4v*>(tw + r * SK_TROW + 64 * h + 16 * p);
      if constexpr (kFused) {
        // k past the range multiplies zero weights: the offset is only kept
        // inside this row's bytes
        const int ka0 = (wave + 4 * (c0 + d)) * 128 + 64 * h;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const int off = min(ka0 + 16 * p, kstride - 16);
          const i32x4v v = *reinterpret_cast<const i32x4v*>(xa + (r < M ? r : 0) * kstride + off);
          am[p] = r < M ? v : i32x4v{};
        }
      } else {
#pragma unroll
        for (int p = 0; p < 4; ++p) am[p] = aq[kFused ? 0 : d][p];
      }
#pragma unroll
      for (int p = 0; p < 4; ++p) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(am[p], bm[p], acc, 0, 0, 0);
      load(c0 + d + SK_D, bq[d], aq[kFused ? 0 : d]);
    }
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) red[wave][i][lane] = acc[i];
  __syncthreads();
  // wave v finishes registers 4v .. 4v+3: rows 8v + 4h + (0..3)
  const int col = n0 + r;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = 4 * wave + q;
    const int row = 8 * wave + 4 * h + q;
    if (row >= M || col >= N) continue;
    const int32_t a = red[0][i][lane] + red[1][i][lane] + red[2][i][lane] + red[3][i][lane];
    if (gridDim.y == 1)
      y[(int64_t)row * N + col] = ((float)a * (kFused ? xsl[row] : xs[row])) * ws[col];
    else
      part[((int64_t)blockIdx.y * M + row) * N + col] = a;
  }
}

// Prefill GEMM (M > 32): a workgroup owns a 128 x 128 output tile, wave
// (wm, wn) the 64 x 64 block at (64 wm, 64 wn) as 2 x 2 MFMA blocks of 32 x
// 32.  K runs in 128-deep chunks: the next chunk's 32 KB (128 rows of A and
// of B, 128 B each: 8 loads of 16 B per thread) is loaded into registers
// while the current one feeds 16 MFMAs per wave from one LDS buffer, then
// stored to the other buffer; one barrier per chunk.  Buffer loads bounded by M*K and
// N*K read rows past M or N and k past the range as zeros.
constexpr int BG_T = 128;
constexpr int BG_KC = 128;
constexpr int BG_LS = BG_KC + 16;  // LDS bytes per staged row
constexpr int BG_SEGS = BG_KC / 16;                 // 16-byte pieces per staged row
constexpr int BG_PIECES = BG_T * BG_SEGS / 256;     // pieces per thread per operand

__global__ __launch_bounds__(256) void int8_gemm_big_kernel(const int8_t* __restrict__ xq,
                                                            const float* __restrict__ xs,
                                                            const int8_t* __restrict__ w,
                                                            const float* __restrict__ ws, float* __restrict__ y,
                                                            int32_t* __restrict__ part, int M, int N, int64_t K,
                                                            int64_t kper) {
  __shared__ __align__(16) int8_t As[2][BG_T * BG_LS];
  __shared__ __align__(16) int8_t Bs[2][BG_T * BG_LS];
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave >> 1, wn = wave & 1, r = lane & 31, h = lane >> 5;
  const int m0 = blockIdx.y * BG_T, n0 = blockIdx.x * BG_T;
  const int64_t kb = (int64_t)blockIdx.z * kper, ke = kb + kper < K ? kb + kper : K;
  constexpr uint32_t kOut = 0x80000000u;
  const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc((void*)xq, (short)0, (int)(M * K), 0x00020000);
  const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, (int)(N * K), 0x00020000);
  // staging: piece p of thread t is row (t + 256 p) / BG_SEGS, bytes 16 * ((t + 256 p) % BG_SEGS)
  uint32_t arow[BG_PIECES], brow[BG_PIECES];
  int prow[BG_PIECES], pseg[BG_PIECES];
#pragma unroll
  for (int p = 0; p < BG_PIECES; ++p) {
    const int id = t + 256 * p;
    prow[p] = id / BG_SEGS;
    pseg[p] = 16 * (id % BG_SEGS);
    arow[p] = m0 + prow[p] < M ? (uint32_t)((int64_t)(m0 + prow[p]) * K) : kOut;
    brow[p] = n0 + prow[p] < N ? (uint32_t)((int64_t)(n0 + prow[p]) * K) : kOut;
  }
  i32x4v ra[BG_PIECES], rb[BG_PIECES];
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int p = 0; p < BG_PIECES; ++p) {
      const uint32_t kk = (uint32_t)(k0 + pseg[p]);
      const bool ok = kk < (uint32_t)ke;  // ke is a multiple of 16
      ra[p] = __builtin_amdgcn_raw_buffer_load_b128(ar, ok ? arow[p] + kk : kOut, 0, 0);
      rb[p] = __builtin_amdgcn_raw_buffer_load_b128(br, ok ? brow[p] + kk : kOut, 0, 0);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int p = 0; p < BG_PIECES; ++p) {
      *reinterpret_cast<i32x4v*>(&As[buf][prow[p] * BG_LS + pseg[p]]) = ra[p];
      *reinterpret_cast<i32x4v*>(&Bs[buf][prow[p] * BG_LS + pseg[p]]) = rb[p];
    }
  };
  gload(kb);
  lstore(0);
  __syncthreads();
  i32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = i32x16{};
  int buf = 0;
  for (int64_t k0 = kb; k0 < ke; k0 += BG_KC) {
    const bool more = k0 + BG_KC < ke;
    if (more) gload(k0 + BG_KC);
#pragma unroll
    for (int s = 0; s < BG_KC / 32; ++s) {
      i32x4v af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        af[i] = *reinterpret_cast<const i32x4v*>(&As[buf][(wm * 64 + i * 32 + r) * BG_LS + 32 * s + 16 * h]);
        bf[i] = *reinterpret_cast<const i32x4v*>(&Bs[buf][(wn * 64 + i * 32 + r) * BG_LS + 32 * s + 16 * h]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (more) lstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + j * 32 + r;
      if (col >= N) continue;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (q / 4) + 4 * h + (q % 4);
        if (row >= M) continue;
        if (gridDim.z == 1)
          y[(int64_t)row * N + col] = ((float)acc[i][j][q] * xs[row]) * ws[col];
        else
          part[((int64_t)blockIdx.z * M + row) * N + col] = acc[i][j][q];
      }
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

constexpr int I8_SKINNY_M = 32;

// K splits for an M x N problem.  Tiled kernel: enough workgroups to cover
// the compute units about twice, each split at least 512 deep.  Skinny
// kernel: up to 2048 waves (8 per compute unit), each split at least 512
// deep (one chunk per wave).
bool int8_skinny(int64_t M, int64_t K, int64_t N) { return M <= I8_SKINNY_M && N * K < ((int64_t)1 << 31); }

// the 128 x 128 prefill kernel: buffer offsets must fit 31 bits
bool int8_big(int64_t M, int64_t K, int64_t N) {
  return M > I8_SKINNY_M && M * K < ((int64_t)1 << 31) && N * K < ((int64_t)1 << 31);
}

int int8_splits(int64_t M, int64_t K, int64_t N) {
  if (K == 0 || K % 16 != 0) return 1;
  int64_t s = 1;
  if (int8_skinny(M, K, N)) {
    const int64_t waves = cdiv(N, 32) * 4;
    while (waves * s * 2 <= 2048 && K / (2 * s) >= 512 && s < 64) s *= 2;
    return (int)s;
  }
  const int64_t bt = int8_big(M, K, N) ? BG_T : I8_BT;
  const int64_t tiles = cdiv(M, bt) * cdiv(N, bt);
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
  hipStream_t st = as_stream(stream);
  const dim3 grid((unsigned)M), block(256);
  if (K % 4 == 0 && K > 0 && aligned(x, 16) && aligned(xq, 4)) {
    const int64_t n4 = K / 4;
    if (n4 <= 256)
      launch(int8_act_quant_vec_kernel<1>, grid, block, 0, st, x, xq, x_scale, K);
    else if (n4 <= 512)
      launch(int8_act_quant_vec_kernel<2>, grid, block, 0, st, x, xq, x_scale, K);
    else if (n4 <= 1024)
      launch(int8_act_quant_vec_kernel<4>, grid, block, 0, st, x, xq, x_scale, K);
    else if (n4 <= 2048)
      launch(int8_act_quant_vec_kernel<8>, grid, block, 0, st, x, xq, x_scale, K);
    else if (n4 <= 4096)
      launch(int8_act_quant_vec_kernel<16>, grid, block, 0, st, x, xq, x_scale, K);
    else
      launch(int8_act_quant_kernel, grid, block, 0, st, x, xq, x_scale, K);
  } else {
    launch(int8_act_quant_kernel, grid, block, 0, st, x, xq, x_scale, K);
  }
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
    launch(int8_gemm_scalar_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st, xq, x_scale, w,
                       w_scale, y, (int)M, (int)N, K);
    return launch_status("ccq_int8_linear");
  }
  const int s = int8_splits(M, K, N);
  const size_t need = ccq_int8_linear_workspace_size(M, K, N);
  CCQ_REQUIRE(s == 1 || (workspace && workspace_bytes >= need && aligned(workspace, 16)),
              "ccq_int8_linear: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  CCQ_REQUIRE(cdiv(M, I8_BT) <= 65535, "ccq_int8_linear: M=%lld too large", (long long)M);
  int nsplit;
  if (int8_skinny(M, K, N)) {
    const int64_t kper = cdiv(cdiv(K, s), 16) * 16;
    nsplit = (int)cdiv(K, kper);
    CCQ_REQUIRE(cdiv(N, 32) <= 0x7fffffff, "ccq_int8_linear: N too large");
    launch(int8_gemm_skinny_kernel<false>, dim3((unsigned)cdiv(N, 32), (unsigned)nsplit), dim3(256), 0,
                       st, xq, (const float*)nullptr, (float*)nullptr, x_scale, w, w_scale, y, (int32_t*)workspace,
                       (int)M, (int)N, K, kper);
  } else if (int8_big(M, K, N)) {
    const int64_t kper = cdiv(cdiv(K, s), BG_KC) * BG_KC;
    const dim3 grid((unsigned)cdiv(N, BG_T), (unsigned)cdiv(M, BG_T), (unsigned)cdiv(K, kper));
    CCQ_REQUIRE(grid.y <= 65535, "ccq_int8_linear: M=%lld too large", (long long)M);
    nsplit = (int)grid.z;
    launch(int8_gemm_big_kernel, grid, dim3(256), 0, st, xq, x_scale, w, w_scale, y,
                       (int32_t*)workspace, (int)M, (int)N, K, kper);
  } else {
    const int64_t kper = cdiv(cdiv(K, s), I8_KC) * I8_KC;
    const dim3 grid((unsigned)cdiv(N, I8_BT), (unsigned)cdiv(M, I8_BT), (unsigned)cdiv(K, kper));
    nsplit = (int)grid.z;
    launch(int8_gemm_kernel, grid, dim3(256), 0, st, xq, x_scale, w, w_scale, y, (int32_t*)workspace,
                       (int)M, (int)N, K, kper);
  }
  if (nsplit > 1)
    launch(int8_splitk_epilogue_kernel, dim3((unsigned)cdiv(M * N, 256)), dim3(256), 0, st,
                       (const int32_t*)workspace, x_scale, w_scale, y, (int)M, (int)N, nsplit);
  return launch_status("ccq_int8_linear");
}

static bool int8_fused_ok(int64_t M, int64_t K, int64_t N) {
  if (M < 1 || M > I8_FUSED_M || K <= 0 || K % 16 != 0 || !int8_skinny(M, K, N)) return false;
  const int64_t kper = cdiv(cdiv(K, int8_splits(M, K, N)), 16) * 16;
  return M * kper <= I8_FUSED_XA;
}

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

extern "C" size_t ccq_int8_w8a8_workspace_size(int64_t M, int64_t K, int64_t N) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  if (int8_fused_ok(M, K, N)) return ccq_int8_linear_workspace_size(M, K, N);
  return align256((size_t)M * (size_t)K) + ccq_int8_linear_workspace_size(M, K, N);
}

extern "C" int ccq_int8_w8a8_linear(const float* x, float* x_scale, const int8_t* w, const float* w_scale, float* y,
                                    int64_t M, int64_t K, int64_t N, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  CCQ_REQUIRE(M >= 0 && K >= 0 && N >= 0, "ccq_int8_w8a8_linear: negative shape");
  CCQ_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff, "ccq_int8_w8a8_linear: M or N too large");
  CCQ_REQUIRE(K < (1 << 17), "ccq_int8_w8a8_linear: K=%lld >= 131072 could overflow the int32 sums", (long long)K);
  if (M == 0) return 0;
  CCQ_REQUIRE(K > 0, "ccq_int8_w8a8_linear: K=0 (a per-token amax over no columns is undefined)");
  CCQ_REQUIRE(x && x_scale && w_scale && y && (w || N == 0), "ccq_int8_w8a8_linear: null pointer");
  const size_t need = ccq_int8_w8a8_workspace_size(M, K, N);
  CCQ_REQUIRE(need == 0 || (workspace && workspace_bytes >= need && aligned(workspace, 256)),
              "ccq_int8_w8a8_linear: workspace of %zu bytes (256-byte aligned) needed, %zu given", need,
              workspace_bytes);
  hipStream_t st = as_stream(stream);
  if (N > 0 && int8_fused_ok(M, K, N) && aligned(x, 16) && aligned(w, 16)) {
    const int s = int8_splits(M, K, N);
    const int64_t kper = cdiv(cdiv(K, s), 16) * 16;
    const int nsplit = (int)cdiv(K, kper);
    launch(int8_gemm_skinny_kernel<true>, dim3((unsigned)cdiv(N, 32), (unsigned)nsplit), dim3(256), 0,
                       st, (const int8_t*)nullptr, x, x_scale, (const float*)x_scale, w, w_scale, y,
                       (int32_t*)workspace, (int)M, (int)N, K, kper);
    if (nsplit > 1)
      launch(int8_splitk_epilogue_kernel, dim3((unsigned)cdiv(M * N, 256)), dim3(256), 0, st,
                         (const int32_t*)workspace, x_scale, w_scale, y, (int)M, (int)N, nsplit);
    return launch_status("ccq_int8_w8a8_linear");
  }
  int8_t* xq = static_cast<int8_t*>(workspace);
  if (int rc = ccq_int8_act_quant(x, xq, x_scale, M, K, stream)) return rc;
  if (N == 0) return 0;
  const size_t off = align256((size_t)M * (size_t)K);
  return ccq_int8_linear(xq, x_scale, w, w_scale, y, M, K, N, static_cast<char*>(workspace) + off,
                         workspace_bytes - off, stream);
}

extern "C" int ccq_int8_dequant(const int8_t* w, const float* scale, float* out, int64_t rows, int64_t cols,
                                void* stream) {
  CCQ_REQUIRE(rows >= 0 && cols >= 0, "ccq_int8_dequant: negative shape");
  if (rows == 0 || cols == 0) return 0;
  CCQ_REQUIRE(w && scale && out, "ccq_int8_dequant: null pointer");
  launch(int8_dequant_kernel, dim3(grid_for(rows * cols, 256)), dim3(256), 0, as_stream(stream), w,
                     scale, out, rows, cols);
  return launch_status("ccq_int8_dequant");
}
