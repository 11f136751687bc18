// Decoded-weight MFMA linear: y[M, N] = x[M, K] @ W[N, K]^T, float32 in and
// out, for the byte-coded weight formats whose reference layers dequantize W
// to float32 and multiply (Fp8LinearMethod.apply / LinearMethod.apply for
// fp8 and int8 keys, quant/fp8.py:35-42, quant/method.py:100-140; the MX
// formats of MxLinearMethod.apply, quant/mx.py:37-94).  For batches past a
// few rows the streaming kernels re-read W once per pass of batch rows; this
// kernel reads W once for up to 64 rows and runs the products on the
// matrix cores.
//
// Arithmetic.  Each weight is decoded in registers to its exact value in
// bf16: e4m3 codes (4 significant bits) times a power-of-two E8M0 scale,
// int8 codes (8 bits), the reference's 4-bit table values times the E8M0
// scale -- all exact in bf16 while the scaled value stays a normal float.
// Activations are split x = hi + lo with hi = bf16(x), lo = bf16(x - hi)
// (|x - hi - lo| <= 2^-17 |x|), and every k-step runs two MFMAs,
// v_mfma_f32_16x16x32_bf16(hi, W) and (lo, W): products of bf16 values are
// exact in the float32 accumulator, so y carries float32 summation error
// only, in an order of its own.  Row scales (FP8 / INT8 per row) and NVFP4's
// second scale multiply the finished sum, as the streaming kernels do.
//
// Tiling.  A workgroup of 8 waves owns 64 output columns and up to 64 batch
// rows (MT tiles of 16; more rows -> more workgroups along y, each reading W
// again).  K runs in chunks of 256: waves 0-3 take the first 128 k of a
// chunk, waves 4-7 the second, each wave 16 columns, and the two halves'
// partial sums are added at the end through LDS in a fixed order.  Lane l
// of a wave holds column l & 15 and the 32 consecutive k of quarter q =
// l >> 4 of its half; MFMA i of the chunk takes each lane's values
// 8i..8i+7, so its 32 k are a fixed permutation of the chunk's -- the same
// permutation on the activation side, read from LDS.  The activation chunk
// (hi and lo bf16, [16 MT][256]) is staged in LDS, double-buffered, one
// barrier per chunk.  Weights (non-temporal loads), scale bytes and the
// activation chunk are loaded PD chunks ahead into a register ring (PD 2-6,
// wq_depth), so the wait for chunk c leaves chunks c+1..c+PD-1 in flight.
#include "ccq_common.h"

namespace ccq {

constexpr int WQ_KC = 256;                 // k per chunk
constexpr int WQ_CG = 4;                   // 16-column groups per workgroup
constexpr int WQ_THREADS = 512;            // 8 waves: 4 column groups x 2 k halves
// LDS row stride in bf16: rows 4 banks apart (padding 0 measured 3.5x the
// bank-conflict cycles and 91 against 53 us at 64 rows; 16 or 24 the same
// as 8)
constexpr int WQ_RS = WQ_KC + 8;
constexpr int WQ_COLS = 16 * WQ_CG;        // output columns per workgroup

struct WqP {
  const float* x;
  const uint8_t* w;
  const void* scale;  // float [N] (row formats), E8M0 bytes [N, K / G] (MX), or null (MXFP4 only)
  float* y;
  int64_t M, K, N;
  int G;
  float s2;
};

template <int FMT>
struct WqTraits {
  static constexpr int WB = FMT == WQ_MXFP4 ? 1 : 2;      // 16-byte weight pieces per lane and chunk
  static constexpr int KDIV = FMT == WQ_MXFP4 ? 2 : 1;    // k per weight byte
  static constexpr bool MX = FMT == WQ_MXFP8 || FMT == WQ_MXFP4;
};

__device__ __forceinline__ bf16x8 pack_bf16x8(const float (&v)[8]) {
  u32x4 r;
  r[0] = bf16x2_bits(v[0], v[1]);
  r[1] = bf16x2_bits(v[2], v[3]);
  r[2] = bf16x2_bits(v[4], v[5]);
  r[3] = bf16x2_bits(v[6], v[7]);
  return __builtin_bit_cast(bf16x8, r);
}

// The lane's weight values 8i..8i+7 of the chunk (times the group scale s
// for the MX formats) as the MFMA's B fragment.
template <int FMT>
__device__ __forceinline__ bf16x8 wq_decode(const u32x4 (&wr)[WqTraits<FMT>::WB], int i, float s) {
  float v[8];
  if constexpr (FMT == WQ_MXFP4) {
    mx4_word(wr[0][i], v);
  } else {
    const uint32_t w0 = wr[i >> 1][(i & 1) * 2], w1 = wr[i >> 1][(i & 1) * 2 + 1];
    if constexpr (FMT == WQ_INT8_ROW) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[j] = (float)(int8_t)(w0 >> (8 * j));
        v[4 + j] = (float)(int8_t)(w1 >> (8 * j));
      }
    } else {
      const auto a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w0, false);
      const auto b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w0, true);
      const auto c = __builtin_amdgcn_cvt_pk_f32_fp8((int)w1, false);
      const auto d = __builtin_amdgcn_cvt_pk_f32_fp8((int)w1, true);
      v[0] = a[0], v[1] = a[1], v[2] = b[0], v[3] = b[1];
      v[4] = c[0], v[5] = c[1], v[6] = d[0], v[7] = d[1];
    }
  }
  if constexpr (WqTraits<FMT>::MX) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] *= s;
  }
  return pack_bf16x8(v);
}

// Scale bytes of MXFP4 layers without scales: E8M0 127 (scale 1), read at
// offset 0, so that every chunk issues the same loads.
__device__ const uint8_t wq_unit_scale[4] = {127, 127, 127, 127};

// Ring loads as inline assembly, so that the compiler adds no waits of its
// own for them (its waits drain every load at the loop head); wq_wait then
// waits for one chunk's loads and wq_tie hands each register of the slot to
// the compiler after that wait.  check_inflight.py verifies on the register
// allocator's output that no instruction reads, copies or spills a ring
// register while its load is in flight.
__device__ __forceinline__ void wq_load16(u32x4& dst, const void* p) {
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(dst) : "v"(p));
}
__device__ __forceinline__ void wq_load_u8(uint32_t& dst, const void* p) {
  asm volatile("global_load_ubyte %0, %1, off" : "=v"(dst) : "v"(p));
}
template <int N>
__device__ __forceinline__ void wq_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// vmcnt(PD - 1 chunks of B + nx loads) for a wave-uniform nx in [0, NX]
template <int PD, int B, int NX>
__device__ __forceinline__ void wq_wait_nx(int nx) {
  if (nx == NX) {
    wq_wait<(PD - 1) * (B + NX)>();
  } else if constexpr (NX > 0) {
    wq_wait_nx<PD, B, NX - 1>(nx);
  } else {
    wq_wait<0>();
  }
}
template <typename T>
__device__ __forceinline__ void wq_tie(T& r) {
  asm volatile("" : "+v"(r));
}

template <int FMT, int MT, int PD, bool G16>
__global__ __launch_bounds__(WQ_THREADS) void wq_mfma_kernel(const WqP p) {
  using Tr = WqTraits<FMT>;
  constexpr int XR = 2 * MT;                        // activation 16-byte pieces per thread and chunk
  constexpr int NSC = Tr::MX ? (G16 ? 2 : 1) : 0;   // scale bytes per lane and chunk
  constexpr int LPC = Tr::WB + NSC + XR;            // loads per lane and chunk
  static_assert((PD - 1) * LPC < 64, "loads in flight fit vmcnt");
  __shared__ __align__(16) uint16_t Xh[2][16 * MT][WQ_RS];
  __shared__ __align__(16) uint16_t Xl[2][16 * MT][WQ_RS];
  __shared__ __align__(16) f32x4 red[WQ_CG][MT][64];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = wave & 3, kh = wave >> 2;
  const int c16 = lane & 15, q = lane >> 4;
  const int64_t M = p.M, K = p.K, N = p.N;
  const int64_t n = (int64_t)blockIdx.x * WQ_COLS + 16 * cg + c16;
  const int64_t m0 = (int64_t)blockIdx.y * 16 * MT;
  const int nch = (int)(K / WQ_KC);
  const int64_t row_bytes = K / Tr::KDIV;
  const uint8_t* wrow = p.w + imin64(n, N - 1) * row_bytes;  // columns past N read row N-1, never stored
  const int lane_k = kh * (WQ_KC / 2) + q * 32;             // first k of the lane's 32 in a chunk
  const bool has_sc = Tr::MX && p.scale != nullptr;
  const int G = G16 ? 16 : 32;
  const uint8_t* srow = has_sc ? reinterpret_cast<const uint8_t*>(p.scale) + imin64(n, N - 1) * (K / G) : wq_unit_scale;

  u32x4 wr[PD][Tr::WB];
  uint32_t sr[PD][NSC > 0 ? NSC : 1];
  u32x4 xr[PD][XR];

  // activation piece j of a thread is row wave + 8j of the tile (wave-
  // uniform): pieces of rows past M are not loaded (zeroed when staged), so
  // a wave issues LPC - XR + nx loads per chunk, nx its valid pieces
  int nx = 0;
#pragma unroll
  for (int j = 0; j < XR; ++j) nx += m0 + wave + 8 * j < M ? 1 : 0;
  auto issue = [&](int s, int c) {
    const int64_t kb = (int64_t)c * WQ_KC;
    const uint8_t* wp = wrow + (kb + lane_k) / Tr::KDIV;
    gload16_nt<0>(wr[s][0], wp);
    if constexpr (Tr::WB == 2) gload16_nt<16>(wr[s][1], wp);
    if constexpr (NSC > 0) {
      const uint8_t* sp = srow + (has_sc ? (kb + lane_k) / G : 0);
      wq_load_u8(sr[s][0], sp);
      if constexpr (NSC == 2) wq_load_u8(sr[s][1], sp + (has_sc ? 1 : 0));
    }
#pragma unroll
    for (int j = 0; j < XR; ++j) {
      const int row = wave + 8 * j, col4 = tid & 63;
      if (j < nx) wq_load16(xr[s][j], p.x + (m0 + row) * K + kb + 4 * col4);
    }
  };
  auto wait_slot = [&](int s, bool steady) {
    if (steady)
      wq_wait_nx<PD, LPC - XR, XR>(nx);
    else
      wq_wait<0>();
#pragma unroll
    for (int j = 0; j < Tr::WB; ++j) wq_tie(wr[s][j]);
#pragma unroll
    for (int j = 0; j < NSC; ++j) wq_tie(sr[s][j]);
#pragma unroll
    for (int j = 0; j < XR; ++j) wq_tie(xr[s][j]);
  };
  auto stage_x = [&](int s, int buf) {
#pragma unroll
    for (int j = 0; j < XR; ++j) {
      const int idx = tid + WQ_THREADS * j, row = idx >> 6, col4 = idx & 63;
      float4 v = __builtin_bit_cast(float4, xr[s][j]);
      if (m0 + row >= M) v = make_float4(0.f, 0.f, 0.f, 0.f);
      const uint32_t h01 = bf16x2_bits(v.x, v.y), h23 = bf16x2_bits(v.z, v.w);
      const uint32_t l01 = bf16x2_bits(v.x - __uint_as_float(h01 << 16), v.y - __uint_as_float(h01 & 0xffff0000u));
      const uint32_t l23 = bf16x2_bits(v.z - __uint_as_float(h23 << 16), v.w - __uint_as_float(h23 & 0xffff0000u));
      *reinterpret_cast<u32x2*>(&Xh[buf][row][4 * col4]) = u32x2{h01, h23};
      *reinterpret_cast<u32x2*>(&Xl[buf][row][4 * col4]) = u32x2{l01, l23};
    }
  };

  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int s = 0; s < PD; ++s)
    if (s < nch) issue(s, s);

  for (int c0 = 0; c0 < nch; c0 += PD) {
#pragma unroll
    for (int s = 0; s < PD; ++s) {
      const int c = c0 + s;
      if (c < nch) {
        const int buf = c & 1;
        wait_slot(s, c + PD - 1 < nch);  // steady: chunks c+1..c+PD-1 were issued after chunk c
        stage_x(s, buf);
        lds_barrier();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float sc = 1.f;
          if constexpr (Tr::MX) sc = e8m0_to_f32(sr[s][NSC == 2 ? (i >> 1) : 0] & 255u);
          const bf16x8 b = wq_decode<FMT>(wr[s], i, sc);
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            const bf16x8 ah = *reinterpret_cast<const bf16x8*>(&Xh[buf][16 * t + c16][lane_k + 8 * i]);
            const bf16x8 al = *reinterpret_cast<const bf16x8*>(&Xl[buf][16 * t + c16][lane_k + 8 * i]);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, b, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, b, acc[t], 0, 0, 0);
          }
        }
        if (c + PD < nch) issue(s, c + PD);
      }
    }
  }

  // second k half -> LDS; the first adds it (fixed order) and stores
  if (kh == 1)
#pragma unroll
    for (int t = 0; t < MT; ++t) red[cg][t][lane] = acc[t];
  __syncthreads();
  if (kh == 0 && n < N) {
    float f = 1.f;
    if constexpr (FMT == WQ_FP8_ROW || FMT == WQ_INT8_ROW) f = reinterpret_cast<const float*>(p.scale)[n];
    if constexpr (FMT == WQ_MXFP4) f = p.s2;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const f32x4 o = red[cg][t][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t r = m0 + 16 * t + 4 * q + i;
        if (r < M) {
          const float v = acc[t][i] + o[i];
          p.y[r * N + n] = (FMT == WQ_MXFP8) ? v : v * f;
        }
      }
    }
  }
}

// Ring depth (chunks loaded ahead) per row-tile count: as deep as the
// registers allow without spills (INT8's decode needs more registers).
template <int FMT, int MT>
constexpr int wq_depth() {
  return FMT == WQ_INT8_ROW ? (MT == 1 ? 4 : (MT == 2 ? 3 : 2)) : (MT == 1 ? 6 : (MT == 2 ? 4 : 3));
}

template <int FMT, bool G16>
static void wq_launch(int mt, const WqP& p, hipStream_t st) {
  const dim3 grid((unsigned)cdiv(p.N, WQ_COLS), (unsigned)cdiv(p.M, 16 * mt));
  if (mt == 1)
    launch((wq_mfma_kernel<FMT, 1, wq_depth<FMT, 1>(), G16>), grid, dim3(WQ_THREADS), 0, st, p);
  else if (mt == 2)
    launch((wq_mfma_kernel<FMT, 2, wq_depth<FMT, 2>(), G16>), grid, dim3(WQ_THREADS), 0, st, p);
  else
    launch((wq_mfma_kernel<FMT, 4, wq_depth<FMT, 4>(), G16>), grid, dim3(WQ_THREADS), 0, st, p);
}

int wq_mfma_linear(int fmt, const float* x, const uint8_t* w, const void* scale, int group_size, float scale2,
                   float* y, int64_t M, int64_t K, int64_t N, hipStream_t stream, const char* name) {
  const bool mx = fmt == WQ_MXFP8 || fmt == WQ_MXFP4;
  if (fmt < WQ_FP8_ROW || fmt > WQ_MXFP4) return -1;
  if (M <= 0 || N <= 0 || K <= 0 || K % WQ_KC != 0) return -1;
  if (!x || !w || !y || !aligned(x, 16) || !aligned(w, 16)) return -1;
  if (!mx && !scale) return -1;
  if (fmt == WQ_MXFP8 && !scale) return -1;
  if (mx && scale && group_size != 16 && group_size != 32) return -1;
  if (cdiv(M, 64) > 65535 || cdiv(N, WQ_COLS) > 0x7fffffff) return -1;
  const int mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const WqP p{x, w, scale, y, M, K, N, mx && scale ? group_size : 32, scale2};
  const bool g16 = mx && scale && group_size == 16;
  switch (fmt) {
    case WQ_FP8_ROW: wq_launch<WQ_FP8_ROW, false>(mt, p, stream); break;
    case WQ_INT8_ROW: wq_launch<WQ_INT8_ROW, false>(mt, p, stream); break;
    case WQ_MXFP8:
      if (g16)
        wq_launch<WQ_MXFP8, true>(mt, p, stream);
      else
        wq_launch<WQ_MXFP8, false>(mt, p, stream);
      break;
    default:
      if (g16)
        wq_launch<WQ_MXFP4, true>(mt, p, stream);
      else
        wq_launch<WQ_MXFP4, false>(mt, p, stream);
      break;
  }
  return launch_status(name);
}

}  // namespace ccq

using namespace ccq;

extern "C" int ccq_wq_mfma_linear_f32(const float* x, const uint8_t* w, const void* scale, float* y, int64_t batch,
                                      int64_t in_features, int64_t out_features, int fmt, int group_size,
                                      float scale2, void* stream) {
  CCQ_REQUIRE(fmt >= WQ_FP8_ROW && fmt <= WQ_MXFP4, "ccq_wq_mfma_linear_f32: fmt=%d (0 fp8 row, 1 int8 row, 2 MXFP8, 3 MXFP4)", fmt);
  CCQ_REQUIRE(batch >= 0 && in_features >= 0 && out_features >= 0, "ccq_wq_mfma_linear_f32: negative shape");
  if (batch == 0 || out_features == 0) return 0;
  CCQ_REQUIRE(x && w && y, "ccq_wq_mfma_linear_f32: null pointer");
  CCQ_REQUIRE(in_features > 0 && in_features % WQ_KC == 0, "ccq_wq_mfma_linear_f32: in_features=%lld must be a positive multiple of %d",
              (long long)in_features, WQ_KC);
  CCQ_REQUIRE(aligned(x, 16) && aligned(w, 16), "ccq_wq_mfma_linear_f32: x and w must be 16-byte aligned");
  CCQ_REQUIRE(fmt == WQ_MXFP4 || scale, "ccq_wq_mfma_linear_f32: fmt %d needs its scales", fmt);
  CCQ_REQUIRE(fmt < WQ_MXFP8 || !scale || group_size == 16 || group_size == 32,
              "ccq_wq_mfma_linear_f32: group_size=%d (16 or 32)", group_size);
  CCQ_REQUIRE(cdiv(batch, 64) <= 65535, "ccq_wq_mfma_linear_f32: batch too large");
  return wq_mfma_linear(fmt, x, w, scale, group_size, scale2, y, batch, in_features, out_features,
                        as_stream(stream), "ccq_wq_mfma_linear_f32");
}
