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


// ---------------------------------------------------------------------------
// Grouped form for MoE experts in the layout the reference's checkpoints and
// ExpertReader hold them (experts/reader.py:142-251): per expert, e4m3 codes
// [out, in] with one float32 scale per output row (BF16 [out, 1] in the
// checkpoint), read in place -- each lane's 32 consecutive k bytes of a row
// are the row-major layout already.  The stage computes, for the tokens
// routed to each expert, the reference's expert_ffn (blocks/moe.py:122-141)
// on the dequantized weights:
//   DUAL (gate/up): y[a, n] = silu(s_g[n] * x_t . Wg[n]) * (s_u[n] * x_t . Wu[n])
//   down:           y[a, n] = s_d[n] * h_a . Wd[n]
// with x_t the float32 row of token t = a / row_div (gate/up) or the
// intermediate row of assignment a (down), in the decoded-weight arithmetic
// above (exact bf16 products of hi/lo activations, float32 accumulation).
// The SiLU product is formed in float64 and rounded once, as the
// reference's silu_mul_fused (quant/kernels.py:219-231).
//
// Grid: x = column blocks of 16*CG columns, y = tiles of the expert-sorted
// schedule (ccq_moe_align with tile_m = 16*MT; tiles past meta[0] exit at
// once).  The 8 waves are CG column groups x KH k parts; a chunk is KH*128 k
// (KH = 2: the dense kernel's 64 columns x 256 k; KH = 4: 32 columns x 512 k,
// KH = 8: 16 columns x 1024 k, for schedules too small to fill the chip
// with wider blocks).  The
// valid rows of a tile are a prefix (an expert's rows are padded at the
// end), so a wave loads only the activation pieces of valid rows and
// zeroes the rest when staging; the k parts' partial sums are added in a
// fixed order through the (then free) activation LDS.
struct WqMoeP {
  const float* x;             // activation rows, K floats each
  const int32_t* rows;        // expert-sorted assignment ids per tile row, -1 = padding
  const int32_t* tile_expert;
  const int32_t* meta;        // meta[0] = tiles in the schedule
  const uint8_t* w0;          // [E][N][K] e4m3 codes: gate (DUAL) or down
  const uint8_t* w1;          // [E][N][K] e4m3 codes: up (DUAL)
  const float* s0;            // [E][N] row scales of w0
  const float* s1;            // [E][N] row scales of w1
  float* y;                   // [assignments][N]
  int64_t N, K;
  int row_div;                // activation row of assignment a = a / row_div
};

// WPE: waves per SIMD the registers must allow (4: two workgroups per CU)
template <bool DUAL, int MT, int PD, int KH, int CW, int WPE = 1>
__global__ __launch_bounds__(WQ_THREADS, WPE) void wq_moe_kernel(const WqMoeP p) {
  constexpr int CG = 8 / KH;                // 16-column groups of waves per workgroup
  constexpr int KC = 128 * KH;              // k per chunk
  constexpr int RS = KC + 8;                // LDS row stride in bf16
  constexpr int TM = 16 * MT;               // rows per tile
  constexpr int NW = DUAL ? 2 : 1;          // weight matrices
  constexpr int NM = NW * CW;               // (matrix, column group) fragments per wave
  constexpr int COLS = 16 * CG * CW;        // columns per workgroup
  constexpr int C4 = KC / 4;                // float4 pieces per activation row and chunk
  constexpr int XR = TM * C4 / WQ_THREADS;  // activation pieces per thread and chunk
  constexpr int LPC = 2 * NM + XR;          // loads per lane and chunk
  static_assert(KH == 2 || KH == 4 || KH == 8, "k parts");
  static_assert(CW == 1 || CW == 2, "column groups per wave");
  static_assert(XR >= 1 && TM * C4 == XR * WQ_THREADS, "activation pieces");
  static_assert(C4 % 64 == 0, "a wave's pieces lie in one row");
  static_assert((PD - 1) * LPC < 64, "loads in flight fit vmcnt");
  static_assert(NM * CG * (KH - 1) * MT * 64 * 16 <= 2 * 2 * TM * RS * 2, "partial sums fit the activation LDS");
  __shared__ __align__(16) uint16_t X[2][2][TM][RS];  // [buffer][hi, lo][row][k]

  const int tile = blockIdx.y;
  if (tile >= p.meta[0]) return;  // uniform: the whole workgroup leaves before any barrier
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = wave % CG, kh = wave / CG;
  const int c16 = lane & 15, q = lane >> 4;
  const int64_t N = p.N, K = p.K;
  const int e = p.tile_expert[tile];
  // column group c of the wave: column (block * COLS) + c * 16 * CG + 16 * cg + c16
  int64_t ncol[CW];
#pragma unroll
  for (int c = 0; c < CW; ++c) ncol[c] = (int64_t)blockIdx.x * COLS + c * 16 * CG + 16 * cg + c16;
  const int nch = (int)(K / KC);
  const int lane_k = kh * 128 + q * 32;  // first k of the lane's 32 in a chunk
  // fragment m = w * CW + c: matrix w (gate / up, or down), column group c;
  // columns past N read row N-1, never stored
  const uint8_t* wrow[NM];
#pragma unroll
  for (int w = 0; w < NW; ++w)
#pragma unroll
    for (int c = 0; c < CW; ++c)
      wrow[w * CW + c] = (w == 0 ? p.w0 : p.w1) + (int64_t)e * N * K + imin64(ncol[c], N - 1) * K + lane_k;
  const int32_t* trow = p.rows + (int64_t)tile * TM;

  // activation piece j of a thread: row (64 wave + 512 j) / C4 of the tile
  // (wave-uniform), float4 column (64 wave + lane + 512 j) % C4; a padding
  // row points at row 0 (in bounds) and is zeroed when staged
  const float* xp[XR];
  uint32_t vmask = 0;
  int nx = 0;
#pragma unroll
  for (int j = 0; j < XR; ++j) {
    const int row = (64 * wave + WQ_THREADS * j) / C4;
    const int a = trow[row];
    if (a >= 0) {
      vmask |= 1u << j;
      nx = j + 1;
    }
    xp[j] = p.x + (int64_t)(a >= 0 ? a / p.row_div : 0) * K + 4 * ((64 * wave + lane + WQ_THREADS * j) % C4);
  }

  u32x4 wr[PD][NM][2];
  u32x4 xr[PD][XR];
  auto issue = [&](int s, int c) {
    const int64_t kb = (int64_t)c * KC;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      gload16_nt<0>(wr[s][m][0], wrow[m] + kb);
      gload16_nt<16>(wr[s][m][1], wrow[m] + kb);
    }
#pragma unroll
    for (int j = 0; j < XR; ++j)
      if (j < nx) wq_load16(xr[s][j], xp[j] + kb);
  };
  auto wait_slot = [&](int s, bool steady) {
    if (steady)
      wq_wait_nx<PD, 2 * NM, XR>(nx);
    else
      wq_wait<0>();
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      wq_tie(wr[s][m][0]);
      wq_tie(wr[s][m][1]);
    }
#pragma unroll
    for (int j = 0; j < XR; ++j) wq_tie(xr[s][j]);
  };
  auto stage_x = [&](int s, int buf) {
#pragma unroll
    for (int j = 0; j < XR; ++j) {
      const int idx = tid + WQ_THREADS * j, row = idx / C4, col4 = idx % C4;
      float4 v = __builtin_bit_cast(float4, xr[s][j]);
      if (!((vmask >> j) & 1u)) v = make_float4(0.f, 0.f, 0.f, 0.f);
      const uint32_t h01 = bf16x2_bits(v.x, v.y), h23 = bf16x2_bits(v.z, v.w);
      const uint32_t l01 = bf16x2_bits(v.x - __uint_as_float(h01 << 16), v.y - __uint_as_float(h01 & 0xffff0000u));
      const uint32_t l23 = bf16x2_bits(v.z - __uint_as_float(h23 << 16), v.w - __uint_as_float(h23 & 0xffff0000u));
      *reinterpret_cast<u32x2*>(&X[buf][0][row][4 * col4]) = u32x2{h01, h23};
      *reinterpret_cast<u32x2*>(&X[buf][1][row][4 * col4]) = u32x2{l01, l23};
    }
  };

  f32x4 acc[NM][MT];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[m][t] = f32x4{0.f, 0.f, 0.f, 0.f};

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
          bf16x8 b[NM];
#pragma unroll
          for (int m = 0; m < NM; ++m) b[m] = wq_decode<WQ_FP8_ROW>(wr[s][m], i, 1.f);
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            const bf16x8 ah = *reinterpret_cast<const bf16x8*>(&X[buf][0][16 * t + c16][lane_k + 8 * i]);
            const bf16x8 al = *reinterpret_cast<const bf16x8*>(&X[buf][1][16 * t + c16][lane_k + 8 * i]);
#pragma unroll
            for (int m = 0; m < NM; ++m) {
              acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, b[m], acc[m][t], 0, 0, 0);
              acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, b[m], acc[m][t], 0, 0, 0);
            }
          }
        }
        if (c + PD < nch) issue(s, c + PD);
      }
    }
  }

  // k parts 1..KH-1 -> LDS (the activation buffers are free once every wave
  // is past its last chunk); part 0 adds them in order and finishes
  __syncthreads();
  f32x4* red = reinterpret_cast<f32x4*>(&X[0][0][0][0]);
  auto red_at = [&](int m, int part, int t) -> f32x4& {
    return red[(((m * CG + cg) * (KH - 1) + part) * MT + t) * 64 + lane];
  };
  if (kh > 0) {
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int t = 0; t < MT; ++t) red_at(m, kh - 1, t) = acc[m][t];
  }
  __syncthreads();
  if (kh != 0) return;
#pragma unroll
  for (int part = 0; part < KH - 1; ++part)
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[m][t] += red_at(m, part, t);
#pragma unroll
  for (int c = 0; c < CW; ++c) {
    const int64_t n = ncol[c];
    if (n >= N) continue;
    const float sc0 = p.s0[(int64_t)e * N + n];
    const float sc1 = DUAL ? p.s1[(int64_t)e * N + n] : 0.f;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int a = trow[16 * t + 4 * q + i];
        if (a < 0) continue;
        float v;
        if constexpr (DUAL) {
          const double g = (double)(acc[c][t][i] * sc0), u = (double)(acc[CW + c][t][i] * sc1);
          v = (float)(g / (1.0 + exp(-g)) * u);
        } else {
          v = acc[c][t][i] * sc0;
        }
        p.y[(int64_t)a * N + n] = v;
      }
  }
}

// Ring depth per row-tile count and fragments per wave.
template <bool DUAL, int MT, int CW>
constexpr int wq_moe_depth() {
  return (DUAL ? 2 : 1) * CW == 1 ? (MT == 1 ? 6 : (MT == 2 ? 4 : 3))
         : (DUAL ? 2 : 1) * CW == 2 ? (MT == 1 ? 4 : (MT == 2 ? 3 : 2))
                                    : (MT <= 2 ? 3 : 2);
}

// cw = 2 (128-column workgroups: each staged activation chunk feeds twice
// the weights) for tiles of 32+ rows, except the gate/up stage's 64-row
// tiles (its registers would spill); 16-row tiles keep narrow workgroups
// (more of them for the few experts of a decode batch)
// A stage whose K is at most two chunks (the down stage, K = inter = 512)
// runs with a 2-deep ring and registers for two workgroups per CU: each
// workgroup's life is about one load latency, so the CU needs two of them.
template <bool DUAL>
static int wq_moe_launch(const WqMoeP& p, int mt, int kh, int64_t max_tiles, hipStream_t st) {
  const int cw = (mt == 2 || (!DUAL && mt == 4)) ? 2 : 1;
  const dim3 grid((unsigned)cdiv(p.N, 16 * (8 / kh) * cw), (unsigned)max_tiles);
#define CCQ_WQM(MT_, KH_, CW_) \
  launch((wq_moe_kernel<DUAL, MT_, wq_moe_depth<DUAL, MT_, CW_>(), KH_, CW_>), grid, dim3(WQ_THREADS), 0, st, p)
#define CCQ_WQS(MT_, KH_, CW_) \
  launch((wq_moe_kernel<false, MT_, 2, KH_, CW_, 4>), grid, dim3(WQ_THREADS), 0, st, p)
  if constexpr (!DUAL) {
    if (p.K <= 2 * 128 * kh) {
      if (mt == 1 && kh == 4)
        CCQ_WQS(1, 4, 1);
      else if (mt == 1)
        CCQ_WQS(1, 2, 1);
      else if (mt == 2)
        CCQ_WQS(2, 2, 2);
      else
        CCQ_WQS(4, 2, 2);
      return launch_status("moe_fp8row down");
    }
  }
  if (mt == 1 && kh == 8 && DUAL)  // 16-column blocks, 1024-k chunks: the few experts of a tiny batch
    launch((wq_moe_kernel<true, 1, 2, 8, 1>), grid, dim3(WQ_THREADS), 0, st, p);
  else if (mt == 1 && kh == 4)
    CCQ_WQM(1, 4, 1);
  else if (mt == 1 && DUAL)  // 16-row gate/up tiles: a 3-deep ring, two workgroups per CU
    launch((wq_moe_kernel<true, 1, 3, 2, 1, 4>), grid, dim3(WQ_THREADS), 0, st, p);
  else if (mt == 1)
    CCQ_WQM(1, 2, 1);
  else if (mt == 2)
    CCQ_WQM(2, 2, 2);
  else if constexpr (DUAL)
    CCQ_WQM(4, 2, 1);
  else
    CCQ_WQM(4, 2, 2);
#undef CCQ_WQM
#undef CCQ_WQS
  return launch_status(DUAL ? "moe_fp8row gate_up" : "moe_fp8row down");
}

// ------------------------------------------------------------ MoE host --
namespace {

struct F8RowLayout {
  int64_t n, max_tiles;
  int mt, kh_gate_up, kh_down;
  size_t off_sorted, off_tile_expert, off_meta, off_counts, off_inter, off_rows, off_align, total;
};

size_t a256(size_t b) { return (b + 255) & ~(size_t)255; }

int device_cus_now() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    return 256;
  return n;
}

// Tile height from the mean rows per routed expert: 16-row tiles for decode
// batches, 32 or 64 when experts hold more rows (each tile reads its
// expert's weights once).  32-column blocks (KH = 4) when 64-column blocks
// would leave most compute units idle.
F8RowLayout f8row_layout(int64_t T, int64_t k, const ccq_fp8row_experts* ex, bool with_cus) {
  F8RowLayout L = {};
  const int64_t E = ex->num_experts, H = ex->hidden, I = ex->inter;
  L.n = T * k;
  const int64_t routed = L.n < E ? L.n : E;
  const int64_t avg = cdiv(L.n, routed > 0 ? routed : 1);
  L.mt = avg <= 8 ? 1 : (avg <= 24 ? 2 : 4);
  const int64_t tile_m = 16 * L.mt;
  L.max_tiles = ccq_moe_align_max_tiles(L.n, E, tile_m);
  const int64_t cus = with_cus ? device_cus_now() : 256;
  L.kh_gate_up = (L.mt == 1 && H % 512 == 0 && cdiv(I, 64) * routed < 2 * cus) ? 4 : 2;
  if (L.kh_gate_up == 4 && H % 1024 == 0 && cdiv(I, 32) * routed < 2 * cus) L.kh_gate_up = 8;
  L.kh_down = (L.mt == 1 && I % 512 == 0 && cdiv(H, 64) * routed < 2 * cus) ? 4 : 2;
  size_t o = 0;
  L.off_sorted = o;
  o += a256((size_t)L.max_tiles * tile_m * 4);
  L.off_tile_expert = o;
  o += a256((size_t)L.max_tiles * 4);
  L.off_meta = o;
  o += 256;
  L.off_counts = o;
  o += a256((size_t)E * 4);
  L.off_inter = o;
  o += a256((size_t)L.n * I * 4);
  L.off_rows = o;
  o += a256((size_t)L.n * H * 4);
  L.off_align = o;
  o += a256(align_scratch_bytes(L.n, E));
  L.total = o;
  return L;
}

int check_fp8row_experts(const ccq_fp8row_experts* ex, const char* name) {
  CCQ_REQUIRE(ex != nullptr, "%s: null experts descriptor", name);
  CCQ_REQUIRE(ex->num_experts >= 1 && ex->num_experts <= 1024, "%s: num_experts=%lld outside [1, 1024]", name,
              (long long)ex->num_experts);
  CCQ_REQUIRE(ex->hidden > 0 && ex->hidden % WQ_KC == 0 && ex->inter > 0 && ex->inter % WQ_KC == 0,
              "%s: hidden=%lld and inter=%lld must be positive multiples of %d", name, (long long)ex->hidden,
              (long long)ex->inter, WQ_KC);
  CCQ_REQUIRE(ex->w_gate && ex->w_up && ex->w_down && ex->s_gate && ex->s_up && ex->s_down,
              "%s: null expert weight or scale pointer", name);
  CCQ_REQUIRE(aligned(ex->w_gate, 16) && aligned(ex->w_up, 16) && aligned(ex->w_down, 16),
              "%s: expert weights must be 16-byte aligned", name);
  return 0;
}

int moe_fp8row_ffn(const float* x, const int64_t* ids, const float* weights, void* y, int y_dtype, int64_t T,
                   int64_t k, const ccq_fp8row_experts* ex, void* workspace, size_t workspace_bytes, void* stream,
                   const float* shared, float shared_gate, const char* name) {
  int rc = check_fp8row_experts(ex, name);
  if (rc) return rc;
  CCQ_REQUIRE(T >= 0 && T <= 65535 && k >= 1 && k <= ex->num_experts, "%s: bad T=%lld / k=%lld", name,
              (long long)T, (long long)k);
  CCQ_REQUIRE(T * k <= 65536, "%s: T*k=%lld > 65536", name, (long long)(T * k));
  CCQ_REQUIRE(y_dtype == CCQ_F32 || y_dtype == CCQ_F16 || y_dtype == CCQ_BF16, "%s: bad y_dtype %d", name, y_dtype);
  if (T == 0) return 0;
  CCQ_REQUIRE(x && ids && weights && y, "%s: null pointer", name);
  CCQ_REQUIRE(aligned(x, 16), "%s: x must be 16-byte aligned", name);
  const F8RowLayout L = f8row_layout(T, k, ex, true);
  CCQ_REQUIRE(L.max_tiles >= 1 && L.max_tiles <= 65535, "%s: %lld tiles exceed the grid", name,
              (long long)L.max_tiles);
  CCQ_REQUIRE(workspace && workspace_bytes >= L.total && aligned(workspace, 256),
              "%s: workspace of %zu bytes (256-byte aligned) needed, %zu given", name, L.total, workspace_bytes);
  hipStream_t st = as_stream(stream);
  char* ws = (char*)workspace;
  int32_t* sorted = (int32_t*)(ws + L.off_sorted);
  int32_t* tile_expert = (int32_t*)(ws + L.off_tile_expert);
  int32_t* meta = (int32_t*)(ws + L.off_meta);
  int32_t* counts = (int32_t*)(ws + L.off_counts);
  float* inter = (float*)(ws + L.off_inter);
  float* rows = (float*)(ws + L.off_rows);
  const int64_t E = ex->num_experts, H = ex->hidden, I = ex->inter;
  rc = launch_align(ids, L.n, E, 16 * L.mt, sorted, tile_expert, meta, counts, st, ws + L.off_align,
                    L.total - L.off_align);
  if (rc) return rc;
  WqMoeP g = {x, sorted, tile_expert, meta, ex->w_gate, ex->w_up, ex->s_gate, ex->s_up, inter, I, H, (int)k};
  rc = wq_moe_launch<true>(g, L.mt, L.kh_gate_up, L.max_tiles, st);
  if (rc) return rc;
  WqMoeP d = {inter, sorted, tile_expert, meta, ex->w_down, nullptr, ex->s_down, nullptr, rows, H, I, 1};
  rc = wq_moe_launch<false>(d, L.mt, L.kh_down, L.max_tiles, st);
  if (rc) return rc;
  return launch_combine(rows, CCQ_F32, weights, ids, E, y, y_dtype, T, k, H, st, shared, shared_gate);
}

}  // namespace

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

extern "C" size_t ccq_moe_fp8row_workspace_size(int64_t T, int64_t k, const ccq_fp8row_experts* ex) {
  if (T <= 0 || k <= 0 || check_fp8row_experts(ex, "ccq_moe_fp8row_workspace_size") != 0) return 0;
  return f8row_layout(T, k, ex, false).total;
}

extern "C" int ccq_moe_fp8row_ffn(const float* x, const int64_t* ids, const float* weights, void* y, int y_dtype,
                                  int64_t T, int64_t k, const ccq_fp8row_experts* ex, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  return moe_fp8row_ffn(x, ids, weights, y, y_dtype, T, k, ex, workspace, workspace_bytes, stream, nullptr, 0.f,
                        "ccq_moe_fp8row_ffn");
}

extern "C" int ccq_moe_fp8row_ffn_shared(const float* x, const int64_t* ids, const float* weights,
                                         const float* shared, float shared_gate, void* y, int y_dtype, int64_t T,
                                         int64_t k, const ccq_fp8row_experts* ex, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  CCQ_REQUIRE(shared || T == 0, "ccq_moe_fp8row_ffn_shared: null shared");
  return moe_fp8row_ffn(x, ids, weights, y, y_dtype, T, k, ex, workspace, workspace_bytes, stream, shared,
                        shared_gate, "ccq_moe_fp8row_ffn_shared");
}
