// AWQ int4 on gfx950: dequant, re-pack into MFMA-ready tiles, the skinny
// (decode) GEMM and the MoE expert FFN built on it.
//
// Weight tile layout ("T16x128"): W[K, N] (in x out) is stored as tiles of
// 128 K-rows x 16 N-columns, tile (kt, nt) at dword offset ((nt*KT + kt)*64 +
// lane)*4, i.e. 1 KiB per tile, one 16-byte slice per lane.  Dword j of lane l
// holds the 8 nibbles of column n = nt*16 + (l & 15) at
// k = kt*128 + 32*j + 8*(l >> 4) + e, e = 0..7, element e in nibble
// (e even ? e/2 : 4 + e/2).  With that order
//     ((dword >> 4r) & 0x000F000F) | MAGIC        r = 0..3
// yields the (e = 2r, 2r+1) pair of the B operand of
// v_mfma_f32_16x16x32_{bf16,f16} as two 16-bit values MAGIC + q, where MAGIC
// is 128 (bf16 0x4300) or 1024 (fp16 0x6400) -- one VALU op per two weights.
// A wave-wide 16-byte load of one tile is a fully coalesced 1 KiB transfer
// that feeds 4 MFMAs (K = 4 x 32).
//
// Scale/zero layout ("SZ"): one 32-bit word per (column, group), scale bits
// (fp16 or bf16) in the low half and the 4-bit zero point in the high half,
// stored column-major: sz[n][g], each column padded to a whole number of
// 4-k-tile chunks (ccq_awq_sz_words).  A lane fetches the scales and zeros of
// its column for 4 k-tiles with one 16-byte load, and no cache line is shared
// between column tiles (so none is fetched twice by different XCDs).
//
// Per quantization group the kernel accumulates
//     tmp = sum_k x[m,k] * (MAGIC + q[k,n])
//     acc += s[g,n] * (tmp - (MAGIC + z[g,n]) * Sx[m,g]),  Sx = sum_k x[m,k]
// which equals sum_k x * (q - z) * s exactly up to float32 rounding; Sx comes
// from one extra MFMA against a ones operand, already in the accumulator
// layout.
#include "ccq_common.h"
#include "ccq_topk.h"

#include <math.h>

#include <mutex>
#include <type_traits>

namespace ccq {

// shift of column 8c + j inside an AWQ word: 4 * AWQ_REVERSE_ORDER[j]
__device__ __forceinline__ int awq_shift(int j) { return 4 * ((j >> 1) + 4 * (j & 1)); }
// nibble slot of element e (k offset 0..7) inside a tile dword
__device__ __forceinline__ int tile_nib(int e) { return (e & 1) ? 4 + (e >> 1) : (e >> 1); }

__device__ __forceinline__ float scale_at(const uint16_t* s, int64_t i, int bf16) {
  uint32_t b = s[i];
  return bf16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

__host__ __device__ inline int64_t sz_words_per_column(int64_t K, int64_t G) {
  return ((K / 128 + 3) / 4) * 4 * (128 / G);
}

// ------------------------------------------------------------------ dequant --
__global__ void awq_dequant_kernel(const uint32_t* __restrict__ qw, const uint32_t* __restrict__ qz,
                                   const uint16_t* __restrict__ sc, int sbf16, float* __restrict__ out,
                                   int64_t K, int64_t N, int64_t G) {
  const int64_t N8 = N / 8, words = K * N8;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t k = i / N8, c = i - k * N8, g = k / G;
    const uint32_t w = qw[i], z = qz[g * N8 + c];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int sh = awq_shift(j);
      const int q = (int)((w >> sh) & 15u) - (int)((z >> sh) & 15u);
      // |q - z| <= 15 times an 11-bit significand: the float32 product is exact
      out[k * N + 8 * c + j] = (float)q * scale_at(sc, g * N + 8 * c + j, sbf16);
    }
  }
}

__global__ void awq_repack_kernel(const uint32_t* __restrict__ qw, uint32_t* __restrict__ tiled, int64_t K,
                                  int64_t N) {
  const int64_t KT = K / 128, N8 = N / 8, total = (N / 16) * KT * 256;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int j = (int)(idx & 3), l = (int)((idx >> 2) & 63);
    const int64_t tile = idx >> 8, kt = tile % KT, nt = tile / KT;
    const int64_t n = nt * 16 + (l & 15);
    const int sh = awq_shift((int)(n & 7));
    const int64_t kb = kt * 128 + 32 * j + 8 * (l >> 4);
    uint32_t o = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) o |= ((qw[(kb + e) * N8 + (n >> 3)] >> sh) & 15u) << (4 * tile_nib(e));
    tiled[idx] = o;
  }
}

__global__ void awq_unpack_tiled_kernel(const uint32_t* __restrict__ tiled, uint32_t* __restrict__ qw, int64_t K,
                                        int64_t N) {
  const int64_t KT = K / 128, N8 = N / 8, words = K * N8;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t k = i / N8, c = i - k * N8, kt = k >> 7;
    const int kk = (int)(k & 127), js = kk >> 5, lq = (kk >> 3) & 3, e = kk & 7;
    uint32_t o = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t n = 8 * c + j, nt = n >> 4;
      const int l = lq * 16 + (int)(n & 15);
      const uint32_t d = tiled[((nt * KT + kt) * 64 + l) * 4 + js];
      o |= ((d >> (4 * tile_nib(e))) & 15u) << awq_shift(j);
    }
    qw[i] = o;
  }
}

// sz[n][g] = scale bits | zero << 16; padding words (g >= K/G) are 0.
__global__ void awq_pack_sz_kernel(const uint32_t* __restrict__ qz, const uint16_t* __restrict__ sc,
                                   uint32_t* __restrict__ sz, int64_t K, int64_t N, int64_t G) {
  const int64_t groups = K / G, W = sz_words_per_column(K, G), total = N * W, N8 = N / 8;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i / W, g = i - n * W;
    uint32_t o = 0;
    if (g < groups) {
      const uint32_t z = (qz[g * N8 + (n >> 3)] >> awq_shift((int)(n & 7))) & 15u;
      o = (uint32_t)sc[g * N + n] | (z << 16);
    }
    sz[i] = o;
  }
}

// ------------------------------------------------------------- MFMA pieces --
template <typename AT>
struct Act;
template <>
struct Act<__bf16> {
  using vec = bf16x8;
  static constexpr uint32_t kMagic2 = 0x43004300u;  // bf16 128.0 twice
  static constexpr float kMagic = 128.0f;
  static constexpr uint32_t kOne2 = 0x3F803F80u;
};
template <>
struct Act<_Float16> {
  using vec = f16x8;
  static constexpr uint32_t kMagic2 = 0x64006400u;  // fp16 1024.0 twice
  static constexpr float kMagic = 1024.0f;
  static constexpr uint32_t kOne2 = 0x3C003C00u;
};

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// 32x32x16: A lane l = row l & 31, B lane l = column l & 31, both with
// k = 8*(l >> 5) + e; D register i of lane l = (row 8*(i/4) + 4*(l >> 5) + i%4,
// column l & 31).
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <typename AT>
__device__ __forceinline__ typename Act<AT>::vec dq_b(uint32_t w) {
  u32x4 r;
  r[0] = (w & 0x000F000Fu) | Act<AT>::kMagic2;
  r[1] = ((w >> 4) & 0x000F000Fu) | Act<AT>::kMagic2;
  r[2] = ((w >> 8) & 0x000F000Fu) | Act<AT>::kMagic2;
  r[3] = ((w >> 12) & 0x000F000Fu) | Act<AT>::kMagic2;
  return __builtin_bit_cast(typename Act<AT>::vec, r);
}

// dq_b with one v_and_or_b32 per weight pair: the mask and the magic come in
// as run-time values (an SGPR and a VGPR), since a VOP3 op on gfx9 takes no
// literal and (w & literal) | literal would cost two ops.
template <typename AT>
__device__ __forceinline__ typename Act<AT>::vec dq_b3(uint32_t w, uint32_t mask_s, uint32_t magic_v) {
  u32x4 r;
  r[0] = (w & mask_s) | magic_v;
  r[1] = ((w >> 4) & mask_s) | magic_v;
  r[2] = ((w >> 8) & mask_s) | magic_v;
  r[3] = ((w >> 12) & mask_s) | magic_v;
  return __builtin_bit_cast(typename Act<AT>::vec, r);
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

__device__ __forceinline__ void store_val(void* y, int64_t i, float v, int dt) {
  if (dt == CCQ_F32)
    reinterpret_cast<float*>(y)[i] = v;
  else if (dt == CCQ_BF16)
    reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)f32_to_bf16_bits(v);
  else
    reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)f32_to_f16_bits(v);
}

// ---------------------------------------------------------- skinny kernel --
enum { EPI_STORE = 0, EPI_SILU = 1, EPI_ROWS = 2 };

struct SkinnyP {
  const void* x;
  int64_t ldx;
  const int32_t* rows;        // per tile 16 row ids (-1 = padding); null = dense rows
  int row_div;                // activation row = row id / row_div
  const int32_t* tile_expert; // expert of each tile; null = single weight
  const int32_t* meta;        // meta[0] = number of valid tiles; null = gridDim.y
  const uint32_t* w0;
  const uint32_t* sz0;
  const uint32_t* w1;         // second weight (up projection) for EPI_SILU
  const uint32_t* sz1;
  int64_t w_es, sz_es;        // per-expert strides (words)
  void* y;
  int64_t ldy;
  int y_dtype;
  int M, N, K, KT;
  int szw;                    // SZ words per column
  int ktpw;                   // k-tiles per wave (a multiple of KTW)
  int xs_rows;                // activation rows a workgroup may stage in LDS
  int xs_ld;                  // LDS row stride of staged activations (elements)
};

// k-tiles whose packed weights, scales and zeros one wave holds in registers
// at once: all of them are requested before the first multiply.
constexpr int KTW = 4;

template <typename ST>
__device__ __forceinline__ float sz_scale(uint32_t word);
template <>
__device__ __forceinline__ float sz_scale<__bf16>(uint32_t word) {
  return __uint_as_float(word << 16);
}
template <>
__device__ __forceinline__ float sz_scale<_Float16>(uint32_t word) {
  return f16_bits_to_f32(word & 0xFFFFu);
}

// One workgroup job: the 16-row tile `tile` times the 16*NB output columns of
// block `nb`, K split over the W waves (wave w owns k-tiles
// [w*ktpw, (w+1)*ktpw), processed in chunks of KTW).  STAGED: the valid rows
// sit in LDS (rows [0, nrows)) next to an all-zero row at index xs_rows that
// padding lanes read, so the loop has no per-lane branches or selects.
// Otherwise every wave loads its A fragments from global memory.
template <typename AT, typename ST, int NB, int GS, int EPI, bool STAGED>
__device__ __forceinline__ void skinny_job(const SkinnyP& p, char* smem, int tile, int nb, int ex, int rid,
                                           bool rvalid, int nrows) {
  using V = typename Act<AT>::vec;
  constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
  constexpr int NG = 4 / GS;               // quantization groups per 128-row tile
  constexpr int NV = NACC * NB * 4;        // accumulator floats per lane
  // k-tiles held per chunk: KTW, or KTW/2 when several groups per k-tile
  // and accumulators would exceed the register budget (the halved chunk is
  // still a whole number of 16-byte SZ records since NG >= 2 there)
  constexpr int KC = (NG >= 2 && NACC * NB * NG >= 4) ? KTW / 2 : KTW;
  constexpr int SZV = (KC * NG + 3) / 4;   // 16-byte SZ loads per chunk
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int r = lane & 15, kq = lane >> 4;
  const int kt0 = wave * p.ktpw;
  const int kt1 = min(p.KT, kt0 + p.ktpw);

  // weight tiles of column block t: uniform base + 16 bytes per lane
  const uint32_t* wcol[NACC][NB];
  const uint32_t* szl[NACC][NB];
#pragma unroll
  for (int q = 0; q < NACC; ++q) {
    const uint32_t* wbase = (q == 0 ? p.w0 : p.w1) + (int64_t)ex * p.w_es;
    const uint32_t* zbase = (q == 0 ? p.sz0 : p.sz1) + (int64_t)ex * p.sz_es;
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      wcol[q][t] = wbase + (int64_t)(nb * NB + t) * p.KT * 256 + lane * 4;
      szl[q][t] = zbase + (int64_t)((nb * NB + t) * 16 + r) * p.szw;
    }
  }

  u32x4 wv[KC][NACC][NB];
  u32x4 szv[NACC][NB][SZV];
  // every weight and scale/zero load of a chunk at once; tiles past the end
  // of the wave's range re-read its last tile (same addresses, no extra HBM
  // traffic) and contribute with a zero scale; SZ columns are padded to
  // whole chunks
  auto load_w = [&](int c0) {
#pragma unroll
    for (int i = 0; i < KC; ++i) {
      const int kt = min(c0 + i, kt1 - 1);
#pragma unroll
      for (int q = 0; q < NACC; ++q)
#pragma unroll
        for (int t = 0; t < NB; ++t)
          wv[i][q][t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wcol[q][t] + kt * 256));
    }
#pragma unroll
    for (int q = 0; q < NACC; ++q)
#pragma unroll
      for (int t = 0; t < NB; ++t)
#pragma unroll
        for (int v = 0; v < SZV; ++v) szv[q][t][v] = *reinterpret_cast<const u32x4*>(szl[q][t] + c0 * NG + 4 * v);
  };
  // the first chunk's HBM reads are in flight while the activations are staged
  if (kt0 < kt1) load_w(kt0);

  AT* xs = reinterpret_cast<AT*>(smem);
  float* red = reinterpret_cast<float*>(smem + (size_t)(p.xs_rows + 1) * p.xs_ld * sizeof(AT));
  const AT* xl = nullptr;
  const AT* xg = nullptr;
  if constexpr (STAGED) {
    const int chunks = p.K / 8;  // 16-byte pieces per row
    for (int c = threadIdx.x; c < nrows * chunks; c += blockDim.x) {
      const int s = c / chunks, off = c - s * chunks;
      const int srid = __shfl(rid, s, 64);  // lanes 0..15 hold rows 0..15
      const bool sval = p.rows ? srid >= 0 : srid < p.M;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (sval)
        v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const AT*>(p.x) + (int64_t)(srid / p.row_div) * p.ldx +
                                            8 * off);
      *reinterpret_cast<u32x4*>(xs + s * p.xs_ld + 8 * off) = v;
    }
    for (int c = threadIdx.x; c < chunks; c += blockDim.x)
      *reinterpret_cast<u32x4*>(xs + p.xs_rows * p.xs_ld + 8 * c) = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();
    xl = xs + (r < nrows ? r : p.xs_rows) * p.xs_ld + 8 * kq;
  } else {
    xg = reinterpret_cast<const AT*>(p.x) + (int64_t)(rvalid ? rid / p.row_div : 0) * p.ldx + 8 * kq;
  }

  f32x4 acc[NACC][NB];
#pragma unroll
  for (int q = 0; q < NACC; ++q)
#pragma unroll
    for (int t = 0; t < NB; ++t) acc[q][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const u32x4 ones_u = {Act<AT>::kOne2, Act<AT>::kOne2, Act<AT>::kOne2, Act<AT>::kOne2};
  const V ones = __builtin_bit_cast(V, ones_u);
  const u32x4 zero4 = {0u, 0u, 0u, 0u};

  for (int c0 = kt0; c0 < kt1; c0 += KC) {
#pragma unroll
    for (int i = 0; i < KC; ++i) {
      const int kt = min(c0 + i, kt1 - 1);
      const bool live = c0 + i < kt1;
      V a[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (STAGED) {
          a[j] = *reinterpret_cast<const V*>(xl + kt * 128 + 32 * j);
        } else {
          const u32x4 v = *reinterpret_cast<const u32x4*>(xg + (int64_t)kt * 128 + 32 * j);
          a[j] = __builtin_bit_cast(V, rvalid ? v : zero4);
        }
      }
      f32x4 sx[NG];
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        sx[g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jj = 0; jj < GS; ++jj) sx[g] = mfma16(a[g * GS + jj], ones, sx[g]);
      }
#pragma unroll
      for (int q = 0; q < NACC; ++q)
#pragma unroll
        for (int t = 0; t < NB; ++t)
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            f32x4 tmp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int jj = 0; jj < GS; ++jj) tmp = mfma16(a[g * GS + jj], dq_b<AT>(wv[i][q][t][g * GS + jj]), tmp);
            const uint32_t word = szv[q][t][(i * NG + g) >> 2][(i * NG + g) & 3];
            const float s = live ? sz_scale<ST>(word) : 0.f;
            const float c = Act<AT>::kMagic + (float)(word >> 16);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[q][t][e] = fmaf(s, fmaf(-c, sx[g][e], tmp[e]), acc[q][t][e]);
          }
    }
    if (c0 + KC < kt1) load_w(c0 + KC);
  }

  if (W > 1) {
    if (wave > 0) {
      float* dst = red + (size_t)(wave - 1) * NV * 64 + lane;
#pragma unroll
      for (int q = 0; q < NACC; ++q)
#pragma unroll
        for (int t = 0; t < NB; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) dst[((q * NB + t) * 4 + i) * 64] = acc[q][t][i];
    }
    __syncthreads();
    if (wave != 0) return;
    for (int w = 1; w < W; ++w) {
      const float* src = red + (size_t)(w - 1) * NV * 64 + lane;
#pragma unroll
      for (int q = 0; q < NACC; ++q)
#pragma unroll
        for (int t = 0; t < NB; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[q][t][i] += src[((q * NB + t) * 4 + i) * 64];
    }
  }

  // rows held by this lane in the accumulator layout: 4*kq + i
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int orid = __shfl(rid, 4 * kq + i, 64);
    const bool ovalid = p.rows ? orid >= 0 : orid < p.M;
    if (!ovalid) continue;
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const int64_t o = (int64_t)orid * p.ldy + (nb * NB + t) * 16 + r;
      if (EPI == EPI_SILU) {
        const float g = acc[0][t][i], u = acc[NACC - 1][t][i];
        store_val(p.y, o, g / (1.0f + expf(-g)) * u, p.y_dtype);
      } else {
        store_val(p.y, o, acc[0][t][i], p.y_dtype);
      }
    }
  }
}

// Workgroup = W waves (W = blockDim.x / 64) sharing one job (row tile
// blockIdx.y, column block blockIdx.x); the W partial sums are added in wave
// order through LDS (deterministic, no global atomics or fences), and wave 0
// runs the epilogue.  The valid rows of a tile are a prefix (dense rows < M;
// the expert schedule pads at the end); when the rows up to the last valid one
// fit the LDS budget (xs_rows) the workgroup stages them in LDS.
template <typename AT, typename ST, int NB, int GS, int EPI>
__global__ __launch_bounds__(512) void w4_skinny_kernel(const SkinnyP p) {
  extern __shared__ __align__(16) char smem[];
  const int lane = threadIdx.x & 63;
  const int nb = blockIdx.x;
  const int tile = blockIdx.y;
  if (p.meta != nullptr && tile >= p.meta[0]) return;  // whole workgroup
  const int ex = p.tile_expert ? p.tile_expert[tile] : 0;
  const int r = lane & 15;
  int rid;
  bool rvalid;
  if (p.rows) {
    rid = p.rows[tile * 16 + r];
    rvalid = rid >= 0;
  } else {
    rid = tile * 16 + r;
    rvalid = rid < p.M;
  }
  const uint64_t vmask = __ballot(rvalid) & 0xFFFFull;
  const int nrows = vmask ? 64 - __clzll(vmask) : 0;
  if (nrows <= p.xs_rows)
    skinny_job<AT, ST, NB, GS, EPI, true>(p, smem, tile, nb, ex, rid, rvalid, nrows);
  else
    skinny_job<AT, ST, NB, GS, EPI, false>(p, smem, tile, nb, ex, rid, rvalid, nrows);
}

// --------------------------------------------------------------- planning --
struct SkinnyPlan {
  int nb;        // 16-column tiles per job
  int nblocks;   // jobs per row tile
  int waves;     // waves per workgroup (K split)
  int ktpw;      // k-tiles per wave
  int xs_rows;   // activation rows staged in LDS
  int xs_ld;     // their LDS row stride (elements)
  size_t lds;    // dynamic LDS bytes
};

// LDS a workgroup may spend on staged activation rows.
constexpr size_t kStageBytes = 24 * 1024;

// K is split over the waves of a workgroup so that each wave holds one chunk
// of KTW k-tiles (all its weight loads in flight at once); at most 8 waves,
// so K > 8*KTW*128 gives each wave several chunks.  Chunk starts are
// multiples of KTW, the granularity of the padded SZ columns.
static SkinnyPlan plan_skinny(int64_t K, int64_t N, int64_t G, int nacc, int NB) {
  SkinnyPlan pl;
  const int64_t KT = K / 128, NT = N / 16;
  if (G < 64 && NB > 2) NB = 2;  // 4 column tiles x 4 groups would spill
  if (NT % NB) NB = (NT % 2 == 0 && NB > 2) ? 2 : 1;
  pl.nb = NB;
  pl.nblocks = (int)(NT / NB);
  int64_t W = cdiv(KT, KTW);
  if (W > 8) W = 8;
  if (W < 1) W = 1;
  pl.ktpw = (int)(cdiv(cdiv(KT, W), KTW) * KTW);
  pl.waves = (int)cdiv(KT, pl.ktpw);
  pl.xs_ld = (int)(K + 8);  // 16 bytes of padding per row staggers LDS banks
  const size_t row_bytes = (size_t)pl.xs_ld * 2;
  pl.xs_rows = (int)imin64(16, (int64_t)(kStageBytes / row_bytes) - 1);  // + the zero row
  pl.lds = (size_t)(pl.xs_rows + 1) * row_bytes + (size_t)(pl.waves - 1) * nacc * NB * 4 * 64 * sizeof(float);
  return pl;
}

template <typename AT, typename ST, int NB, int EPI>
static void launch_skinny_gs(const SkinnyP& p, dim3 grid, int waves, size_t lds, hipStream_t st, int G) {
  const dim3 block(64 * waves);
  if (G == 128)
    launch((w4_skinny_kernel<AT, ST, NB, 4, EPI>), grid, block, lds, st, p);
  else if (G == 64)
    launch((w4_skinny_kernel<AT, ST, NB, 2, EPI>), grid, block, lds, st, p);
  else if constexpr (NB <= 2)  // plan_skinny never pairs 4 column tiles with G = 32
    launch((w4_skinny_kernel<AT, ST, NB, 1, EPI>), grid, block, lds, st, p);
}

template <typename AT, typename ST, int EPI>
static void launch_skinny_nb(const SkinnyP& p, const SkinnyPlan& pl, dim3 grid, hipStream_t st, int G) {
  if constexpr (EPI != EPI_STORE) {
    launch_skinny_gs<AT, ST, 1, EPI>(p, grid, pl.waves, pl.lds, st, G);
  } else {
    if (pl.nb == 1)
      launch_skinny_gs<AT, ST, 1, EPI>(p, grid, pl.waves, pl.lds, st, G);
    else if (pl.nb == 2)
      launch_skinny_gs<AT, ST, 2, EPI>(p, grid, pl.waves, pl.lds, st, G);
    else
      launch_skinny_gs<AT, ST, 4, EPI>(p, grid, pl.waves, pl.lds, st, G);
  }
}

template <int EPI>
static void launch_skinny(SkinnyP p, int x_bf16, int s_bf16, const SkinnyPlan& pl, int64_t tiles, hipStream_t st,
                          int G) {
  p.ktpw = pl.ktpw;
  p.xs_rows = pl.xs_rows;
  p.xs_ld = pl.xs_ld;
  const dim3 grid((unsigned)pl.nblocks, (unsigned)tiles);
  if (x_bf16) {
    if (s_bf16)
      launch_skinny_nb<__bf16, __bf16, EPI>(p, pl, grid, st, G);
    else
      launch_skinny_nb<__bf16, _Float16, EPI>(p, pl, grid, st, G);
  } else {
    if (s_bf16)
      launch_skinny_nb<_Float16, __bf16, EPI>(p, pl, grid, st, G);
    else
      launch_skinny_nb<_Float16, _Float16, EPI>(p, pl, grid, st, G);
  }
}

// 16-column tiles per job of the dense GEMM: more columns per wave re-use
// each activation fragment over more weights once several rows are valid.
static int gemm_nb(int64_t M) { return M <= 4 ? 1 : (M <= 8 ? 2 : 4); }

static bool valid_group(int64_t G) { return G == 32 || G == 64 || G == 128; }

// ------------------------------------------------ decode streaming GEMM --
// For up to 16 rows per weight (decode; MoE experts receiving a few tokens):
// pure weight streaming.  One persistent workgroup of 8 waves per compute
// unit takes a contiguous range of jobs; a job is one 16-row tile times NQ
// "quads" of 16 output columns over all of K: the gate and the up columns of
// one 16-column block for EPI_SILU, two adjacent 16-column blocks otherwise
// (NQ = 2), or one block (NQ = 1, K up to 4096).  The 8 waves split K (wave w
// takes k-tiles w, w + 8, ...).  Each wave streams its own weight tiles
// (1 KiB per 128 K x 16 columns, one 16-byte slice per lane) and one
// scale/zero word per lane straight into registers, WS_DEPTH jobs ahead, so
// the weight stream needs no LDS and no barrier: with 8 waves that is
// WS_DEPTH x 34 KiB in flight per compute unit.  The tile's activation
// fragments and their group sums (one MFMA against a ones operand) stay in
// registers; the fragments of a second tile in the range wait in LDS.  The
// waves' partial sums go through LDS and are added in a fixed order, two jobs
// per barrier (waves 0..3 add the first, 4..7 the second).  The schedule
// (valid tiles, experts, row ids) is read with scalar loads.
struct W4SP {
  const void* x;
  int64_t ldx;
  const int32_t* rows;         // per tile 16 row ids (-1 = padding); null = dense rows
  int row_div;                 // activation row = row id / row_div
  const int32_t* tile_expert;  // expert of each tile; set exactly when rows is
  const int32_t* meta;         // meta[0] = valid tiles; null = tiles
  int tiles;
  const uint32_t* w0;
  const uint32_t* sz0;
  const uint32_t* w1;          // up projection (EPI_SILU)
  const uint32_t* sz1;
  int64_t w_es, sz_es;         // per-expert strides (words)
  void* y;
  int64_t ldy;
  int y_dtype;
  int M, N, K, KT, szw;
  uint32_t nib_mask;           // 0x000F000F (a run-time value, see dq_b3)
  // routing on the fly (EPI_SILU only): non-null logits [rT, rE] replace
  // rows / tile_expert / meta; every workgroup routes the rT tokens itself
  // and workgroup 0 writes the routing and the schedule for the next kernels
  const float* logits;
  int rT, rE, rk, rmode;
  // 1: the stack holds one more expert (index rE, the shared expert) that
  // every token takes as assignment slot rk with weight rshared_w
  int rshared;
  float rshared_w;
  int64_t* ids_out;            // [rT, rk + rshared]
  float* wts_out;              // [rT, rk + rshared]
  int32_t* sched_rows;         // [tiles * 16], as ccq_moe_align's sorted_ids
  int32_t* sched_tile_expert;  // [tiles]
  int32_t* sched_meta;         // [2]
  int32_t* sched_counts;       // [rE]
  // routed down stage (EPI_ROWS with ROUTE): the assignments' rows of x are
  // the MFMA rows (rT of them, at most 16); rows, tile_expert and meta are the
  // gate/up stage's schedule (tiles = its capacity); every workgroup takes
  // one 16-column block across all tiles and combines the assignments'
  // rows into y [cT, N]: y[t] = sum over slots of cwts[t*ck + s] * row
  // (slots with cids outside [0, cE) skipped), as moe_combine_kernel does
  const float* cwts;
  const int64_t* cids;
  int64_t cE;
  void* cy;
  int64_t ldcy;
  int cy_dtype, cT, ck;
};

// ---- routing of a decode batch inside a workgroup ----
// Top-k of every token (one wave per token, two tokens at once for E <= 64,
// the routing kernel's own code, on logits staged in LDS) and the expert
// schedule of ccq_moe_align with 16-row tiles: experts in first-appearance
// order, each expert's assignments ascending, tiles padded with -1.  One
// wave builds the schedule, lane l holding assignments l, 64 + l, ...
// (chunks of 64): ballots over the expert id bits of each chunk give every
// assignment the lanes holding the same expert, so its rank among them, its
// expert's count and whether it is the expert's first appearance; a scan
// over the first appearances gives the padded bases.  Limits: RT_MAXN
// assignments, RT_MAXE experts, RT_MAXLG logits.
constexpr int RT_MAXN = 256;
constexpr int RT_MAXE = 256;
constexpr int RT_MAXLG = 4096;
constexpr int RT_CHUNKS = RT_MAXN / 64;
constexpr int RT_MAXTILES = RT_MAXN / 16 + RT_MAXN;  // ccq_moe_align_max_tiles(RT_MAXN, .., 16) at most
struct RouteSmem {
  float lg[RT_MAXLG];
  int sid[RT_MAXN];  // expert of each assignment, -1 = dropped
  int cnt[RT_MAXE], base[RT_MAXE], rank_of[RT_MAXE];
  int sorted[RT_MAXTILES * 16];
  int tile_expert[RT_MAXTILES];
  int ntiles, nactive;
};

__device__ __forceinline__ int pad16(int c) { return (c + 15) & ~15; }
__device__ __forceinline__ int popc64(uint64_t m) { return (int)__popcll(m); }
template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_add_src(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, ROWS, 0xf, false);
}
// Inclusive sum over the wave on DPP moves (row_shr 1, 2, 4, 8 within the
// 16-lane rows, then row_bcast 15 and 31 carry the row totals forward):
// no LDS round trip.
__device__ __forceinline__ int wave_incl_sum(int v) {
  v += dpp_add_src<0x111, 0xf>(v);
  v += dpp_add_src<0x112, 0xf>(v);
  v += dpp_add_src<0x114, 0xf>(v);
  v += dpp_add_src<0x118, 0xf>(v);
  v += dpp_add_src<0x142, 0xa>(v);
  v += dpp_add_src<0x143, 0xc>(v);
  return v;
}

constexpr int RT_LGV = RT_MAXLG / 512;  // logits per thread of a 512-thread workgroup

// The batch's logits into registers (thread t: logits t, t + 512, ...).
__device__ __forceinline__ void route_logits_load(const W4SP& p, float (&lgv)[RT_LGV]) {
  const int tid = threadIdx.x, TE = p.rT * p.rE;
#pragma unroll
  for (int j = 0; j < RT_LGV; ++j) lgv[j] = tid + 512 * j < TE ? p.logits[tid + 512 * j] : 0.f;
}

// Top-k of the batch in every workgroup (blockDim.x = 512): the logits
// (from route_logits_load) staged in LDS, rs.sid[a] = expert of assignment
// a (-1: dropped), rs.cnt[e] = assignments of expert e; workgroup 0 writes
// ids and weights out.  LDS-only barriers, so weight loads issued before it
// stay in flight.
__device__ void route_topk(const W4SP& p, RouteSmem& rs, const float (&lgv)[RT_LGV]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  // E logits per token, Es experts in the schedule (E + the shared one),
  // ks assignment slots per token (the shared one last)
  const int T = p.rT, E = p.rE, k = p.rk, ks = k + p.rshared, Es = E + p.rshared;
  for (int e = tid; e < Es; e += blockDim.x) rs.cnt[e] = 0;
#pragma unroll
  for (int j = 0; j < RT_LGV; ++j)
    if (tid + 512 * j < T * E) rs.lg[tid + 512 * j] = lgv[j];
  lds_barrier();
  auto keep = [&](int t, float w, int id) {
    if (lane < k) {
      const int a = t * ks + lane;
      const bool ok = id >= 0 && id < E;
      rs.sid[a] = ok ? id : -1;
      if (ok) atomicAdd(&rs.cnt[id], 1);
      if (blockIdx.x == 0) {
        p.ids_out[a] = id;
        p.wts_out[a] = w;
      }
    } else if (lane == k && p.rshared) {
      const int a = t * ks + k;
      rs.sid[a] = E;
      atomicAdd(&rs.cnt[E], 1);
      if (blockIdx.x == 0) {
        p.ids_out[a] = E;
        p.wts_out[a] = p.rshared_w;
      }
    }
  };
  if (E <= 64) {  // tokens t and t + nw together (a lone last token runs twice)
    for (int t = wave; t < T; t += 2 * nw) {
      const int t2 = t + nw < T ? t + nw : t;
      float w[2];
      int id[2];
      topk_rows<1, 2>(rs.lg + t * E, (int64_t)(t2 - t) * E, E, k, p.rmode, w, id);
      keep(t, w[0], id[0]);
      if (t2 != t) keep(t2, w[1], id[1]);
    }
  } else {
    for (int t = wave; t < T; t += nw) {
      float w;
      int id;
      const float* lr = rs.lg + t * E;
      if (E <= 128)
        topk_row<2>(lr, E, k, p.rmode, w, id);
      else
        topk_row<4>(lr, E, k, p.rmode, w, id);
      keep(t, w, id);
    }
  }
  lds_barrier();
}

// The schedule of ccq_moe_align (16-row tiles) from rs.sid, built by wave 0
// of workgroup 0 and published for the down and combine kernels.  Barriers
// are LDS-only, so the caller's weight loads stay in flight.
__device__ void route_schedule(const W4SP& p, RouteSmem& rs) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = p.rT, k = p.rk, ks = k + p.rshared, Es = p.rE + p.rshared, n = T * ks;
  const int nslots = n + 15 * min(n, Es);  // the padded schedule is at most this long
  for (int i = tid; i < nslots; i += blockDim.x) rs.sorted[i] = -1;
  lds_barrier();
  if (wave == 0) {
    int nbits = 1;
    while ((1 << nbits) < Es) ++nbits;  // <= 8
    const int nch = (n + 63) / 64;     // <= RT_CHUNKS
    const uint64_t lt = (1ull << lane) - 1ull;
    int key[RT_CHUNKS], rank[RT_CHUNKS], cnt[RT_CHUNKS];
    uint64_t vm[RT_CHUNKS];
#pragma unroll
    for (int c = 0; c < RT_CHUNKS; ++c) {
      const int a = 64 * c + lane;
      key[c] = c < nch && a < n ? rs.sid[a] : -1;
      vm[c] = __ballot(key[c] >= 0);
      rank[c] = 0;
      cnt[c] = 0;
    }
    // lanes of chunk d with the expert of this lane's assignment in chunk c
#pragma unroll
    for (int d = 0; d < RT_CHUNKS; ++d) {
      if (d >= nch) break;
      uint64_t bd[8];
#pragma unroll
      for (int b = 0; b < 8; ++b) bd[b] = b < nbits ? __ballot(key[d] >= 0 && ((key[d] >> b) & 1)) : 0ull;
#pragma unroll
      for (int c = 0; c < RT_CHUNKS; ++c) {
        if (c >= nch) break;
        uint64_t m = key[c] >= 0 ? vm[d] : 0ull;
#pragma unroll
        for (int b = 0; b < 8; ++b)
          if (b < nbits) m &= ((key[c] >> b) & 1) ? bd[b] : ~bd[b];
        cnt[c] += popc64(m);
        if (d < c) rank[c] += popc64(m);
        if (d == c) rank[c] += popc64(m & lt);
      }
    }
    // first appearances in assignment order: the experts' order, padded
    // sizes and bases (exclusive scan carried across the chunks)
    int carry = 0, nact = 0;
#pragma unroll
    for (int c = 0; c < RT_CHUNKS; ++c) {
      if (c >= nch) break;
      const bool first = key[c] >= 0 && rank[c] == 0;
      const int pd = first ? pad16(cnt[c]) : 0;
      const int incl = wave_incl_sum(pd);
      if (first) {
        const int bs = carry + incl - pd;
        rs.base[key[c]] = bs;
        for (int t = bs / 16; t < (bs + pd) / 16; ++t) rs.tile_expert[t] = key[c];
      }
      carry += __builtin_amdgcn_readlane(incl, 63);
      nact += popc64(__ballot(first));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the bases above, before this wave reads them
#pragma unroll
    for (int c = 0; c < RT_CHUNKS; ++c) {
      if (c >= nch) break;
      if (key[c] >= 0) rs.sorted[rs.base[key[c]] + rank[c]] = 64 * c + lane;
    }
    if (lane == 0) {
      rs.ntiles = carry / 16;
      rs.nactive = nact;
    }
  }
  lds_barrier();
  const int nt = rs.ntiles;
  for (int i = tid; i < nt * 16; i += blockDim.x) p.sched_rows[i] = rs.sorted[i];
  for (int i = tid; i < nt; i += blockDim.x) p.sched_tile_expert[i] = rs.tile_expert[i];
  for (int x = tid; x < Es; x += blockDim.x) p.sched_counts[x] = rs.cnt[x];
  if (tid == 0) {
    p.sched_meta[0] = nt;
    p.sched_meta[1] = rs.nactive;
  }
  lds_barrier();  // every wave has read the scratch before the first job reuses the space
}

constexpr int WS_DEPTH = 2;  // jobs of weights in flight per wave (2 measured faster than 4 or 6)
constexpr int WS_DEPTH_MT1 = 4;  // the same with one k-tile per wave (K <= 1024)
// Routed down stage with the combine: at most RD_MAXA assignments (one
// 16-row MFMA tile), RD_DEPTH jobs in flight per wave (a workgroup's jobs
// are one per routed expert, so all of them at once for up to six experts)
constexpr int RD_MAXA = 16;
constexpr int RD_DEPTH = 6;
constexpr int RT_LEAD = 2;   // jobs workgroup 0 of a routed gate/up stage gives up for building the schedule

// Quads per job of the streaming kernel for a stage of N columns and K rows
// (0: the kernel does not take it).  EPI_SILU always pairs gate and up; two
// quads keep K <= 2048 (two k-tiles per wave), one quad K <= 4096.
static int stream_nq(int EPI, int64_t N, int64_t K, int64_t G) {
  if (G != 128 || K % 128 != 0 || N % 16 != 0) return 0;
  const int64_t KT = K / 128;
  const bool two = EPI == EPI_SILU || N % 32 == 0;
  if (two && KT <= 16) return 2;
  if (EPI != EPI_SILU && KT <= 32) return 1;
  return 0;
}

template <typename AT, typename ST, int EPI, int MT, int NQ, bool ROUTE = false>
__global__ __launch_bounds__(512) void w4_stream_kernel(const W4SP p) {
  using V = typename Act<AT>::vec;
  // routed down stage with the combine (see W4SP): a workgroup's jobs are
  // one column block of each routed expert, all of them in flight at once
  constexpr bool RDOWN = ROUTE && EPI == EPI_ROWS;
  constexpr int D = RDOWN ? RD_DEPTH : (MT == 1 ? WS_DEPTH_MT1 : WS_DEPTH);
  static_assert(MT != 1 || (EPI == EPI_ROWS && !ROUTE), "one k-tile per wave: the down stage on a schedule");
  static_assert(EPI != EPI_SILU || NQ == 2, "gate and up quads");
  static_assert(MT * NQ <= 4, "one scale/zero word per lane covers a wave's share of a job");
  static_assert(D % 2 == 0, "jobs are reduced in pairs");
  constexpr int XB = MT == 2 ? 8 * MT * 4 * 64 : 1;  // second tile's fragments (MT = 4 runs one tile)
  __shared__ __align__(16) f32x4 part[2][2][NQ][8][64];
  __shared__ __align__(16) V xb[XB];
  __shared__ int Rid[2][16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int NJ = p.N / (EPI == EPI_SILU ? 16 : 16 * NQ), KT = p.KT, szw = p.szw;  // jobs per tile
  // the routing scratch lives in the partial-sum buffer, unused until the
  // first job
  RouteSmem& rs = *reinterpret_cast<RouteSmem*>(&part[0][0][0][0][0]);
  static_assert(!ROUTE || EPI == EPI_ROWS || (EPI == EPI_SILU && sizeof(RouteSmem) <= sizeof(part)),
                "routing in gate/up only");
  static_assert(!RDOWN || NQ == 1, "routed down: 16-column blocks");
  constexpr bool routed = ROUTE;  // token (or assignment) rows; p.logits is set exactly for routed gate/up
  const int r16 = lane & 15, kq = lane >> 4;
  // activation fragments, lane r16 holding MFMA row r16.  A routed batch
  // (T <= 16 tokens) multiplies every expert's weights by all its tokens:
  // the MFMA rows are the tokens, the same for every job, so their
  // fragments are loaded once, before the routing, and each job stores
  // only the rows of the tokens routed to its expert.  k-tiles past K
  // repeat the last one (those k-tiles get a zero scale)
  V a[MT][4], b[MT][4];
  auto load_frags = [&](V (&f)[MT][4], int xrow) {
    const AT* xr = reinterpret_cast<const AT*>(p.x) + (int64_t)xrow * p.ldx + 8 * kq;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const int kt = min(wave + 8 * m, KT - 1);
#pragma unroll
      for (int j = 0; j < 4; ++j) f[m][j] = *reinterpret_cast<const V*>(xr + kt * 128 + 32 * j);
    }
  };
  if constexpr (routed) load_frags(a, r16 < p.rT ? r16 : 0);
  // routed: the expert of each job tile and, per token, its assignment in
  // the tile (-1: not routed there), in the second-tile fragment area
  // (unused with token rows)
  int* const ste = reinterpret_cast<int*>(&xb[0]);
  int* const tok2a = ste + RT_MAXTILES;
  float* const rv = reinterpret_cast<float*>(tok2a + RT_MAXTILES * 16);  // routed down: [16 assignments][16 columns]
  float* const cw_s = rv + RD_MAXA * 16;                                   // routed down: slot weights,
  int* const cok_s = reinterpret_cast<int*>(cw_s + RD_MAXA);               // and whether the slot is routed
  static_assert(!ROUTE || (MT == 2 && (RT_MAXTILES * 17 + RD_MAXA * 18) * 4 <= XB * 16),
                "routed tables fit the fragment area");
  // ---- the weight stream: a wave's share of one job is MT x NQ tiles (16 B
  // per lane) and the scale/zero words of its k-tiles for the 16 columns of
  // each quad (lane l: column l & 15, (m, q) pair l >> 4).  Every load is
  // issued unconditionally, so that the compiler's count of loads in flight
  // stays exact and each wait leaves the later jobs' loads in flight: a slot
  // past the end of the range reads the first KiB of the weights (and the
  // first words of the scales) instead, the same lines for every workgroup,
  // which stay in L2 ----
  const int zmq = (lane >> 4) < MT * NQ ? lane >> 4 : 0;
  const int zq = zmq % NQ, zkt = min(wave + 8 * (zmq / NQ), KT - 1);
  // column job nj of expert e_x (real = false: the hot line)
  auto load_ej = [&](int e_x, int nj, bool real, u32x4 (&w)[MT][NQ], uint32_t& z) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const int kt = min(wave + 8 * m, KT - 1);
      const bool live = real && wave + 8 * m < KT;  // k-tiles past K: the hot line too
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const uint32_t* base = EPI == EPI_SILU && q == 1 ? p.w1 : p.w0;
        int64_t off = (int64_t)e_x * p.w_es +
                      ((int64_t)(EPI == EPI_SILU ? nj : nj * NQ + q) * KT + kt) * 256;
        off = live ? off : 0;
        // the select stays on the offset (the compiler would otherwise load
        // from both addresses and select the data); the base keeps the
        // pointer in the global address space
        asm volatile("" : "+s"(off));
        // non-temporal: read once (measured 8% faster than plain loads for the
        // gate/up stage of a 16-token decode batch)
        w[m][q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + off) + lane);
      }
    }
    const uint32_t* zbase = EPI == EPI_SILU && zq == 1 ? p.sz1 : p.sz0;
    int64_t zoff = (int64_t)e_x * p.sz_es + ((int64_t)(EPI == EPI_SILU ? nj : nj * NQ + zq) * 16 + r16) * szw + zkt;
    zoff = real ? zoff : lane;
    asm volatile("" : "+v"(zoff));
    z = zbase[zoff];
  };
  u32x4 wv[D][MT][NQ];
  uint32_t zv[D];

  int ntiles, lead = 0;
  if constexpr (RDOWN) {
    // the gate/up stage's schedule (at most RD_MAXA assignments, so at most
    // that many one-tile experts), read in one round trip up to its
    // capacity: ste[tile] = expert, tok2a[tile][a] = a for its assignments
    const int cap = min(p.tiles, RD_MAXA);
    const int rw = tid < cap * 16 ? p.rows[tid] : -1;
    const int te = tid < cap ? p.tile_expert[tid] : 0;
    // the combine's slot weights and ids, in the same round trip
    const int na = p.cT * p.ck;
    const float cw = tid < na ? p.cwts[tid] : 0.f;
    const int64_t ci = tid < na ? p.cids[tid] : -1;
    ntiles = min(p.meta[0], cap);
    if (tid < na) {
      cw_s[tid] = cw;
      cok_s[tid] = ci >= 0 && ci < p.cE ? 1 : 0;
    }
    for (int i = tid; i < RD_MAXA * 16; i += blockDim.x) tok2a[i] = -1;
    lds_barrier();
    if (tid < ntiles * 16 && rw >= 0 && rw < RD_MAXA) tok2a[(tid >> 4) * 16 + rw] = rw;
    if (tid < ntiles) ste[tid] = te;
    lds_barrier();
  } else if constexpr (routed) {
    // The job tiles are the routed experts in id order (tile r: expert
    // ste[r]), straight from the top-k: the gate/up jobs need no schedule,
    // so the weight loads start right after it.  Workgroup 0 builds the
    // published schedule (first-appearance order) once its loads are in
    // flight, and takes RT_LEAD fewer jobs.
    const int Es = p.rE + p.rshared, na = p.rT * p.row_div;
    float lgv[RT_LGV];
    route_logits_load(p, lgv);
    route_topk(p, rs, lgv);
    for (int i = tid; i < min(na, Es) * 16; i += blockDim.x) tok2a[i] = -1;
    if (wave == 0) {
      int carry = 0;
      for (int c = 0; c < Es; c += 64) {
        const int e = c + lane;
        const bool used = e < Es && rs.cnt[e] > 0;
        const uint64_t m = __ballot(used);
        if (used) {
          const int r = carry + popc64(m & ((1ull << lane) - 1ull));
          rs.rank_of[e] = r;
          ste[r] = e;
        }
        carry += popc64(m);
      }
      if (lane == 0) rs.ntiles = carry;
    }
    lds_barrier();
    for (int i = tid; i < na; i += blockDim.x) {
      const int e = rs.sid[i];
      if (e >= 0) tok2a[rs.rank_of[e] * 16 + i / p.row_div] = i;
    }
    ntiles = __builtin_amdgcn_readfirstlane(rs.ntiles);
    lead = ntiles * NJ >= 4 * (int)gridDim.x ? RT_LEAD : 0;
    lds_barrier();  // every wave has read the routing scratch before the first job reuses the space
  } else {
    ntiles = p.meta != nullptr ? p.meta[0] : p.tiles;
  }
  // jobs of the workgroup: a contiguous range on a schedule (one or two
  // tiles); for dense rows (one tile) every gridDim-th job, so that the
  // workgroups together sweep the weights in address order (measured 7%
  // faster than contiguous ranges on a load-only copy of the stream; for
  // the routed stage, whose consecutive jobs then change experts, 12%
  // slower)
  constexpr bool IL = EPI == EPI_STORE || RDOWN;  // routed down: gridDim.x = column blocks
  const int J = ntiles * NJ;
  // (32-bit: b * (J + lead) < 256 * 2^23 for the schedules this kernel takes)
  auto split = [&](int b) {
    return b == 0 ? 0 : max(0, (int)((uint32_t)b * (uint32_t)(J + lead) / gridDim.x) - lead);
  };
  const int lo = IL ? (int)blockIdx.x : split(blockIdx.x);
  const int hi = IL ? J : split(blockIdx.x + 1);
  // routed down: the combine of moe_combine_kernel for this block's 16
  // columns (slots in order, fmaf, slots of dropped assignments skipped)
  auto combine = [&]() {
    if (tid < p.cT * 16) {
      const int t = tid >> 4, c = tid & 15;
      float acc = 0.f;
      for (int s = 0; s < p.ck; ++s) {
        const int a = t * p.ck + s;
        if (cok_s[a]) acc = fmaf(cw_s[a], rv[a * 16 + c], acc);
      }
      const int64_t o = (int64_t)t * p.ldcy + (int64_t)blockIdx.x * 16 + c;
      if (p.cy_dtype == CCQ_F32)
        reinterpret_cast<float*>(p.cy)[o] = acc;
      else if (p.cy_dtype == CCQ_BF16)
        reinterpret_cast<uint16_t*>(p.cy)[o] = (uint16_t)f32_to_bf16_bits(acc);
      else
        reinterpret_cast<uint16_t*>(p.cy)[o] = (uint16_t)f32_to_f16_bits(acc);
    }
  };
  if (lo >= hi) {
    if constexpr (routed && !RDOWN) {
      if (blockIdx.x == 0) route_schedule(p, rs);
    }
    if constexpr (RDOWN) combine();  // no routed assignment: zeros
    return;
  }
  const int n = RDOWN ? ntiles
                      : (IL ? (hi - lo <= (int)gridDim.x ? 1 : (hi - lo + (int)gridDim.x - 1) / (int)gridDim.x)
                            : hi - lo);
  const int tA = IL ? 0 : lo / NJ, ntl = IL ? 1 : (hi - 1) / NJ - tA + 1;  // the range covers 1 or 2 tiles
  const int tB = ntl > 1 ? tA + 1 : tA;
  auto job_of = [&](int i) { return IL ? lo + i * (int)gridDim.x : lo + i; };
  // a contiguous range covers at most two tiles: job i's tile and column
  // from the range's first column nj0, without a run-time division per job
  const int nj0 = IL ? 0 : lo - tA * NJ;
  auto tile_col = [&](int i, int job, int& tl, int& nj) {
    if constexpr (RDOWN) {  // job i is tile i of this workgroup's column block
      tl = i;
      nj = (int)blockIdx.x;
    } else if constexpr (IL) {
      tl = p.tiles == 1 ? 0 : job / NJ;  // dense rows: usually one tile
      nj = job - tl * NJ;
    } else {
      const int c = nj0 + i;
      tl = c >= NJ ? tA + 1 : tA;
      nj = c >= NJ ? c - NJ : c;
    }
  };

  // ---- experts and row ids of the range's tiles: scalar loads, issued
  // together; lane r16 keeps row r16 ----
  int exA = 0, exB = 0, rid[2] = {-1, -1};
  if (routed) {  // token rows: the tables above
  } else if (p.rows != nullptr) {  // expert schedule (rows and tile_expert both set)
    const int32_t* ra = p.rows + (int64_t)tA * 16;
    const int32_t* rb = p.rows + (int64_t)tB * 16;
    exA = p.tile_expert[tA];
    exB = p.tile_expert[tB];
    int va = -1, vb = -1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int sa = ra[r], sb = rb[r];
      va = r16 == r ? sa : va;
      vb = r16 == r ? sb : vb;
    }
    rid[0] = va;
    rid[1] = vb;
  } else {  // dense rows of one weight
    rid[0] = tA * 16 + r16 < p.M ? tA * 16 + r16 : -1;
    rid[1] = tB * 16 + r16 < p.M ? tB * 16 + r16 : -1;
  }
  if (!routed && wave == 0 && lane < 32) Rid[kq][r16] = kq == 0 ? rid[0] : rid[1];  // read after the first barrier
  const int nvalid0 = (int)__popcll(__ballot(lane < 16 && rid[0] >= 0));
  const int nvalid1 = (int)__popcll(__ballot(lane < 16 && rid[1] >= 0));

  // ---- tile-row fragments (issued before the weights, so that waiting
  // for them does not wait for the weight stream): a padding row reads the
  // tile's first row (padding rows are never stored) ----
  if constexpr (!routed) {
    const int rA = rid[0] >= 0 ? rid[0] : __shfl(rid[0], 0, 64);
    const int rB = rid[1] >= 0 ? rid[1] : __shfl(rid[1], 0, 64);
    const int rd = p.row_div;  // 1 for the down stage: no division
    load_frags(a, rd == 1 ? rA : rA / rd);
    if constexpr (MT <= 2) load_frags(b, rd == 1 ? rB : rB / rd);  // MT = 1: kept in registers
  }

  // routed down: lane l holds the expert of tile l (at most RD_MAXA tiles),
  // so a job's expert is a readlane rather than an LDS round trip
  const int ste_v = RDOWN && lane < ntiles ? ste[lane] : 0;
  auto load = [&](int i, u32x4 (&w)[MT][NQ], uint32_t& z) {
    const bool real = i < n;
    const int job = job_of(real ? i : 0);
    int tl, nj;
    tile_col(real ? i : 0, job, tl, nj);
    const int e_x = RDOWN ? __builtin_amdgcn_readlane(ste_v, tl)
                          : (routed ? __builtin_amdgcn_readfirstlane(ste[tl]) : (tl == tA ? exA : exB));
    load_ej(e_x, nj, real, w, z);
  };
#pragma unroll
  for (int d = 0; d < D; ++d) load(d, wv[d], zv[d]);
  if constexpr (routed && !RDOWN) {
    if (blockIdx.x == 0) route_schedule(p, rs);
  }

  // park the second tile's fragments in LDS, group sums of the first
  if constexpr (MT == 2) {
    if (!routed && ntl > 1) {
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j) xb[((wave * MT + m) * 4 + j) * 64 + lane] = b[m][j];
    }
  }
  const V ones = __builtin_bit_cast(V, u32x4{Act<AT>::kOne2, Act<AT>::kOne2, Act<AT>::kOne2, Act<AT>::kOne2});
  f32x4 sx[MT];
  auto group_sums = [&]() {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      sx[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) sx[m] = mfma16(a[m][j], ones, sx[m]);
    }
  };
  group_sums();

  const uint32_t mask_s = p.nib_mask;
  uint32_t magic_v = Act<AT>::kMagic2;
  asm volatile("v_mov_b32 %0, %0" : "+v"(magic_v));  // keep the magic in a VGPR (far from any MFMA)

  // this wave's share of a job's product (lane: rows 4*kq + i of column r16
  // of each quad), the MT x NQ MFMA chains interleaved, into LDS
  // the first MM of the wave's MT k-tiles, those past K/128 with a zero
  // scale (their loads read the hot line)
  auto compute_mm = [&](auto mm_tag, const u32x4 (&w)[MT][NQ], uint32_t z, int pp, int jj) {
    constexpr int MM = decltype(mm_tag)::value;
    f32x4 t[MT][NQ];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
      for (int q = 0; q < NQ; ++q) t[m][q] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int q = 0; q < NQ; ++q) t[m][q] = mfma16(a[m][j], dq_b3<AT>(w[m][q][j], mask_s, magic_v), t[m][q]);
    f32x4 acc[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const bool live = wave + 8 * m < KT;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const uint32_t zz = (uint32_t)__shfl((int)z, (m * NQ + q) * 16 + r16, 64);
        const float s = live ? sz_scale<ST>(zz) : 0.f, c = Act<AT>::kMagic + (float)(zz >> 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[q][i] = fmaf(s, fmaf(-c, sx[m][i], t[m][q][i]), acc[q][i]);
      }
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) part[pp][jj][q][wave][lane] = acc[q];
  };
  // a wave whose second k-tile lies past K (K/128 not a multiple of 8, two
  // k-tiles per wave) skips its MFMAs, which frees the SIMD for the partner
  // wave
  const bool one_live = MT == 2 && wave + 8 >= KT;  // wave-uniform
  // one k-tile per wave: a wave past K only writes zero partials
  const bool dead = MT == 1 && wave >= KT;
  auto compute = [&](const u32x4 (&w)[MT][NQ], uint32_t z, int pp, int jj) {
    if (dead)
      compute_mm(std::integral_constant<int, 0>{}, w, z, pp, jj);
    else if (one_live)
      compute_mm(std::integral_constant<int, 1>{}, w, z, pp, jj);
    else
      compute_mm(std::integral_constant<int, MT>{}, w, z, pp, jj);
  };

  // sum of the 8 waves' partials of one job (fixed order) and the store;
  // thread u of the half-workgroup holds row 4*(l/16) + i4 of column l%16
  auto reduce = [&](int ii, int pp, int jj) {  // ii: the workgroup's job index
    const int job = job_of(ii);
    int tl, nj;
    tile_col(ii, job, tl, nj);
    const int ts = tl == tA ? 0 : 1;
    const int u = tid & 255, l = u >> 2, i4 = u & 3, row = 4 * (l >> 4) + i4;
    const int orow = routed ? tok2a[tl * 16 + row] : (row < (ts == 0 ? nvalid0 : nvalid1) ? Rid[ts][row] : -1);
    if (orow < 0) return;
    float pv[NQ][8];
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
      for (int w = 0; w < 8; ++w) pv[q][w] = reinterpret_cast<const float*>(&part[pp][jj][q][w][l])[i4];
    float v[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      float s = pv[q][0];
#pragma unroll
      for (int w = 1; w < 8; ++w) s += pv[q][w];
      v[q] = s;
    }
    const int64_t o = (int64_t)orow * p.ldy + (l & 15);
    if constexpr (EPI == EPI_SILU) {
      const float g = v[0], up = v[1];
      store_val(p.y, o + nj * 16, g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * up, p.y_dtype);
    } else if constexpr (RDOWN) {
      (void)o;
      rv[orow * 16 + (l & 15)] = v[0];  // the assignment's row, this block's columns
    } else {
#pragma unroll
      for (int q = 0; q < NQ; ++q) store_val(p.y, o + (nj * NQ + q) * 16, v[q], p.y_dtype);
    }
  };

  // ---- the range's jobs: job i uses register set i % D, and its slot is
  // refilled with job i + D right after; a barrier after every pair.  Whole
  // blocks of D jobs first (loads without conditions), then the rest ----
  const int iB = ntl > 1 ? (tA + 1) * NJ - lo : n;  // first job of the second tile
  auto enter = [&](int i) {
    if constexpr (MT == 2 && !routed) {  // (token rows: the same fragments for every tile)
      if (i == iB) {  // the range moves on to its second tile
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
          for (int j = 0; j < 4; ++j) a[m][j] = xb[((wave * MT + m) * 4 + j) * 64 + lane];
        group_sums();
      }
    } else if constexpr (MT == 1 && !routed) {
      if (i == iB) {
#pragma unroll
        for (int j = 0; j < 4; ++j) a[0][j] = b[0][j];
        group_sums();
      }
    }
  };
  auto pair_done = [&](int i) {  // jobs i - 1 and i are in LDS
    lds_barrier();
    const int jj = wave >> 2;
    if (i - 1 + jj < n) reduce(i - 1 + jj, (i >> 1) & 1, jj);
  };
  const int nfull = n / D * D;
  for (int g = 0; g < nfull; g += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int i = g + d;
      enter(i);
      compute(wv[d], zv[d], (i >> 1) & 1, i & 1);
      load(i + D, wv[d], zv[d]);
      if (d & 1) pair_done(i);
    }
  }
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int i = nfull + d;
    if (i < n) {
      enter(i);
      compute(wv[d], zv[d], (i >> 1) & 1, i & 1);
    }
    if ((d & 1) && i - 1 < n) pair_done(i);
  }
  if constexpr (RDOWN) {
    lds_barrier();  // every job's rows in rv
    combine();
  }
}

// Launch of the streaming kernel; tiles = 16-row tiles the grid is sized for
// (at most one workgroup per compute unit, at most one tile change per range;
// K > 2048 only for a single tile).
template <int EPI>
static int launch_stream(const W4SP& p, int nq, int x_bf16, int s_bf16, int64_t tiles, hipStream_t st);

// ------------------------------------------------ prefill grouped GEMM --
// For tiles with many rows (prefill; experts receiving tens to thousands of
// tokens).  A workgroup of 8 waves computes a 128-row tile against 128
// columns of gate and of up (EPI_SILU) or 128 / 256 columns of one matrix.
// The waves form a 2 (rows) x 4 (columns) grid, each owning 64 rows (two
// 32-row tiles) x C32 tiles of 32 columns on v_mfma_f32_32x32x16, so every
// activation fragment read from LDS feeds C32 MFMAs and every dequantized
// weight fragment two.  Group size 128 is one k-tile; per k-tile
//     acc += s * sum_k x * (MAGIC + q)  -  Sx * s * (MAGIC + z)
// where Sx is the sum of the row's 128 activations of that group, computed
// beforehand (row_group_sums_kernel for a layer input, the gate/up epilogue
// for the intermediate rows).  The second term is a rank-1 update per
// k-tile; two k-tiles' worth go in as one v_mfma_f32_32x32x2f32 (rows' -Sx
// against columns' s * (MAGIC + z)) instead of a VALU FMA per element.
//
// Per k-tile the workgroup copies from HBM straight into LDS
// (global_load_lds, no registers): the activation tile (128 rows x 256 B,
// gathered through the tile's row ids), the packed weight tiles (1 KiB per
// 16 columns), their scale/zero words and the rows' Sx.  Three k-tiles form
// a ring, so two k-tiles of loads are in flight while one is multiplied,
// with a single barrier per k-tile.  Activation rows keep their 16-byte
// pieces XOR-swizzled by row (piece p of row r at position p ^ (r & 15)):
// the MFMA operand reads of 16 consecutive rows then hit 16 different bank
// groups.  Weights are dequantized in registers after the LDS read.
struct W4GP {
  const void* x;
  int64_t ldx;                 // activation row stride (elements)
  const float* sx;             // per-row group sums of x: sx[row * ldsx + kt]
  int64_t ldsx;
  const int32_t* rows;         // per tile 128 row ids (-1 = padding, at the end); null = dense rows
  int row_div;                 // activation row = row id / row_div
  const int32_t* tile_expert;  // null = one weight
  const int32_t* meta;         // meta[0] = valid schedule tiles; null = tiles
  int tiles;
  const uint32_t* w0;
  const uint32_t* sz0;
  const uint32_t* w1;          // up projection (EPI_SILU)
  const uint32_t* sz1;
  int64_t w_es, sz_es;         // per-expert strides (words)
  void* y;
  int64_t ldy;
  int y_dtype;
  float* sxo;                  // EPI_SILU: group sums of the stored rows, sxo[row id * ldsxo + block]
  int64_t ldsxo;
  int M, N, K, KT, szw;
  uint32_t nib_mask;           // 0x000F000F (a run-time value, see dq_b3)
};

constexpr int GG_BM = 128;
constexpr int GG_A_BYTES = GG_BM * 256;  // 128 rows x 128 16-bit activations
constexpr int GG_B_BYTES = 16 * 1024;    // up to 16 packed weight tiles
constexpr int GG_SZ_BYTES = 256 * 4;     // up to 256 scale/zero words
constexpr int GG_SX_BYTES = GG_BM * 4;
constexpr int GG_B_OFF = GG_A_BYTES;
constexpr int GG_SZ_OFF = GG_B_OFF + GG_B_BYTES;
constexpr int GG_SX_OFF = GG_SZ_OFF + GG_SZ_BYTES;
constexpr int GG_STAGE = GG_SX_OFF + GG_SX_BYTES;
constexpr int GG_STAGES = 3;
constexpr int GG_RID = GG_BM + 64;  // row ids of one item + copies of its expert id
static_assert(GG_STAGES * GG_STAGE + 3 * GG_RID * 4 + 4 * GG_BM * 4 <= 160 * 1024, "LDS budget of one workgroup");



template <typename AT, typename ST, int EPI, int CTW>
__global__ __launch_bounds__(512) void w4_group_gemm_kernel(const W4GP p) {
  using V = typename Act<AT>::vec;
  constexpr int NQ = EPI == EPI_SILU ? 2 : 1;
  constexpr int WGN = 64 * CTW;      // columns per matrix per item
  constexpr int TPM = WGN / 16;      // 16-column weight tiles per matrix per k-tile
  constexpr int NBT = NQ * TPM;      // weight tiles per k-tile
  constexpr int BPW = NBT / 8;       // weight tiles each wave copies
  constexpr int NSZ = NQ * WGN;      // scale/zero words per k-tile
  constexpr int C32 = CTW * NQ / 2;  // 32-column MFMA tiles per wave
  constexpr int CQ = C32 / NQ;       // ... per matrix
  static_assert(NBT % 8 == 0 && NBT <= 16 && NSZ <= 256 && NSZ % 64 == 0 && C32 >= 1 && BPW <= 2, "tile shape");
  __shared__ __align__(16) char smem[GG_STAGES * GG_STAGE];
  __shared__ __align__(16) int Rid[3][GG_RID];  // row ids (+ expert id copies) of items j, j+1, j+2
  __shared__ __align__(16) float part[4 * GG_BM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int mw = wave >> 2, nw = wave & 3;
  const int nblk = p.N / WGN;
  const int ntiles = p.meta != nullptr ? p.meta[0] : p.tiles;
  // Static schedule: workgroup b runs on XCD b % 8 (nx workgroups per XCD).
  // Row tiles are dealt to the XCDs round-robin (tile t to XCD t % 8), so an
  // expert with many tiles is spread over all of them, and all column blocks
  // of a tile stay on one XCD, sharing its activations in that L2.  Within
  // an XCD, workgroup wx takes every nx-th of the XCD's items (tile-major).
  const int xcd = blockIdx.x & 7, wx = blockIdx.x >> 3;
  const int nx = ((int)gridDim.x - xcd + 7) >> 3;
  const int items_x = (ntiles > xcd ? (ntiles - xcd + 7) >> 3 : 0) * nblk;
  if (wx >= items_x) return;
  // Items are dealt in rounds of nx, alternating direction: the workgroup
  // that takes a round's first item takes the next round's last.  The
  // schedule lists experts by first appearance, which tends to put the full
  // tiles of often-routed experts early and part-filled tiles late, so the
  // alternation pairs heavy items with light ones (measured against plain
  // round-robin: T=512 top-8 layer, 128 experts, gate/up -5%, down -13%).
  auto item_of = [&](int j) { return j * nx + ((j & 1) ? nx - 1 - wx : wx); };
  const int nmine = items_x / nx + (item_of(items_x / nx) < items_x ? 1 : 0);
  const int KT = p.KT;
  const int total = nmine * KT;  // k-steps of this workgroup

  // ---- row ids: rows of item j go to Rid[j % 3], copied (DMA) at the first
  // k-step of item j - 2; Rid[.][GG_BM..] holds the item's expert ----
  auto tile_of = [&](int j) { return xcd + 8 * (item_of(j) / nblk); };
  auto fetch_rows = [&](int j) {  // waves 5..7
    if (j >= nmine) return;
    const int tile = tile_of(j);
    const uint32_t dst = lds_addr(&Rid[j % 3][0]);
    if (wave >= 6) dma4(p.rows + (int64_t)tile * GG_BM, (wave - 6) * 256 + lane * 4, dst + (wave - 6) * 256);
    if (wave == 5 && p.tile_expert != nullptr) dma4(p.tile_expert + tile, 0u, dst + GG_BM * 4);
  };
  // prologue: items 0 and 1 with plain loads
  for (int j = 0; j < 2 && j < nmine; ++j) {
    const int tile = tile_of(j);
    if (tid < GG_BM) Rid[j][tid] = p.rows[(int64_t)tile * GG_BM + tid];
    if (tid == GG_BM) Rid[j][GG_BM] = p.tile_expert != nullptr ? p.tile_expert[tile] : 0;
  }
  __syncthreads();

  // ---- per-item copy plan of this wave ----
  struct Plan {
    uint32_t aoff[4];
    const char* bsrc[BPW];
    const char* zsrc;
    uint32_t zoff, soff;
    int nvalid, nb;
  };
  const bool has_sz = wave < NSZ / 64;
  const bool has_sx = wave == 4 || wave == 5;
  const int ncopy = 4 + BPW + (has_sz ? 1 : 0) + (has_sx ? 1 : 0);
  auto make_plan = [&](int j, Plan& P) {
    P.nb = item_of(j) % nblk;
    const int* R = Rid[j % 3];
    const int ex = p.tile_expert != nullptr ? __builtin_amdgcn_readfirstlane(R[GG_BM]) : 0;
    // valid rows form a prefix of the tile
    P.nvalid = (int)(__popcll(__ballot(R[lane] >= 0)) + __popcll(__ballot(R[64 + lane] >= 0)));
    const int rid0 = R[0];
    // activations: rows 16*wave + 4*i + (lane >> 4); the lane takes piece
    // (lane & 15) ^ (row & 15), which lands at position lane & 15
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * wave + 4 * i + (lane >> 4);
      const int rid = R[row] >= 0 ? R[row] : rid0;
      const int piece = (lane & 15) ^ (4 * i + (lane >> 4));
      P.aoff[i] = (uint32_t)((int64_t)(rid / p.row_div) * p.ldx * 2 + piece * 16);
    }
#pragma unroll
    for (int b2 = 0; b2 < BPW; ++b2) {
      const int b = wave * BPW + b2, q = b / TPM, nt = P.nb * TPM + (b - q * TPM);
      P.bsrc[b2] = reinterpret_cast<const char*>((q == 0 ? p.w0 : p.w1) + (int64_t)ex * p.w_es + (int64_t)nt * KT * 256);
    }
    P.zsrc = nullptr;
    P.zoff = 0;
    if (has_sz) {
      const int q = (64 * wave) / WGN, col = P.nb * WGN + (64 * wave - q * WGN) + lane;
      P.zoff = (uint32_t)((int64_t)col * p.szw * 4);
      P.zsrc = reinterpret_cast<const char*>((q == 0 ? p.sz0 : p.sz1) + (int64_t)ex * p.sz_es);
    }
    P.soff = 0;
    if (has_sx) {
      const int row = 64 * (wave - 4) + lane;
      const int rid = R[row] >= 0 ? R[row] : rid0;
      P.soff = (uint32_t)((int64_t)(rid / p.row_div) * p.ldsx * 4);
    }
  };
  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](const Plan& P, int kt, int slot) {
    const uint32_t st = lds0 + slot * GG_STAGE;
    const char* xb = reinterpret_cast<const char*>(p.x) + (int64_t)kt * 256;
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(xb, P.aoff[i], st + (16 * wave + 4 * i) * 256);
#pragma unroll
    for (int b2 = 0; b2 < BPW; ++b2)
      dma16_nt(P.bsrc[b2] + (int64_t)kt * 1024, lane * 16, st + GG_B_OFF + (wave * BPW + b2) * 1024);
    if (has_sz) dma4(P.zsrc + kt * 4, P.zoff, st + GG_SZ_OFF + wave * 256);
    if (has_sx) dma4(p.sx + kt, P.soff, st + GG_SX_OFF + (wave - 4) * 256);
  };

  // ---- MFMA side: v_mfma_f32_32x32x16; the wave owns rows mw*64 + 32*rt
  // (rt = 0, 1) and C32 32-column tiles; lane (h, c32) = (lane >> 5, lane & 31) ----
  const int c32 = lane & 31, h = lane >> 5;
  // A operand of k-step s: row c32 of the 32-row tile, piece 2s + h (swizzled)
  uint32_t adoff[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) adoff[s] = (mw * 64 + c32) * 256 + (((2 * s + h) ^ (c32 & 15)) * 16);
  // B operand: column c32 of the tile = column c32 & 15 of 16-column weight
  // tile (c32 >> 4); its k-step s sits in dword s >> 1 of the 16-byte slot
  // of lane 16 * (2 * (s & 1) + h) + (c32 & 15)
  uint32_t bdoff[C32][2];
  uint32_t zdoff[C32];
#pragma unroll
  for (int c = 0; c < C32; ++c) {
    const int q = c / CQ, cc = c - q * CQ;
    const int t16 = q * TPM + nw * CTW + 2 * cc + (c32 >> 4);
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) bdoff[c][pp] = GG_B_OFF + t16 * 1024 + (16 * (2 * pp + h) + (c32 & 15)) * 16;
    zdoff[c] = GG_SZ_OFF + (q * WGN + nw * CTW * 16 + cc * 32 + c32) * 4;
  }
  // Waves of the second row half (sharing SIMDs with the first) fold a
  // k-tile's products at the start of the next one, so the two waves of a
  // SIMD are not in their VALU-only phase at the same time.
  const bool late = mw == 1;

  f32x16 acc[2][C32], t[2][C32];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int c = 0; c < C32; ++c) {
      acc[rt][c] = f32x16{};
      t[rt][c] = f32x16{};
    }
  // zero-point term over windows of 2 groups on the fp32 MFMA (32x32x2):
  // acc -= Sx[row][g] * s[g][col] * (MAGIC + z[g][col]); lane half h holds group 2m + h
  float za[2], zb[C32], sc[C32], scp[C32];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) za[rt] = 0.f;
#pragma unroll
  for (int c = 0; c < C32; ++c) {
    zb[c] = 0.f;
    sc[c] = 0.f;
    scp[c] = 0.f;
  }
  const uint32_t mask_s = p.nib_mask;
  uint32_t magic_v = Act<AT>::kMagic2;
  asm volatile("v_mov_b32 %0, %0" : "+v"(magic_v));  // keep the magic in a VGPR (far from any MFMA)

  // two = the wave's second 32-row tile holds valid rows (wave-uniform;
  // without, its MFMAs, fold and correction are skipped)
  auto fold = [&](const float (&s)[C32], bool two) {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      if (rt == 1 && !two) break;
#pragma unroll
      for (int c = 0; c < C32; ++c)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[rt][c][i] = fmaf(s[c], t[rt][c][i], acc[rt][c][i]);
    }
  };

  // mid (the next copies' issue) runs halfway through the k-step's MFMAs,
  // where its scalar work overlaps the matrix pipe (after the barrier, so
  // the slot it refills is free; measured 3% faster than before the MFMAs)
  auto compute = [&](int slot, int kt, bool two, auto&& mid) {
    const char* S = smem + slot * GG_STAGE;
    const bool mine = h == (kt & 1);
    if (late && (kt & 1)) fold(scp, two);  // products of the even k-tile before
    u32x4 bq[C32][2];
#pragma unroll
    for (int c = 0; c < C32; ++c) {
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) bq[c][pp] = *reinterpret_cast<const u32x4*>(S + bdoff[c][pp]);
      const uint32_t z = *reinterpret_cast<const uint32_t*>(S + zdoff[c]);
      sc[c] = sz_scale<ST>(z);
      const float zc = sc[c] * (Act<AT>::kMagic + (float)(z >> 16));
      zb[c] = mine ? zc : zb[c];
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const float sxr = *reinterpret_cast<const float*>(S + GG_SX_OFF + (mw * 64 + rt * 32 + c32) * 4);
      za[rt] = mine ? -sxr : za[rt];
    }
    // the k-steps in two straight-line forms (one or two 32-row tiles), so no
    // branch splits the dequantization of one fragment from the MFMAs of the
    // one before
    auto ksteps = [&](auto two_c) {
      constexpr bool TWO = decltype(two_c)::value;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        if (s == 4) mid();
        V a[2];
#pragma unroll
        for (int rt = 0; rt < (TWO ? 2 : 1); ++rt) a[rt] = *reinterpret_cast<const V*>(S + rt * 32 * 256 + adoff[s]);
#pragma unroll
        for (int c = 0; c < C32; ++c) {
          const V b = dq_b3<AT>(bq[c][s & 1][s >> 1], mask_s, magic_v);
          t[0][c] = mfma32(a[0], b, s == 0 ? f32x16{} : t[0][c]);
          if constexpr (TWO) t[1][c] = mfma32(a[1], b, s == 0 ? f32x16{} : t[1][c]);
        }
      }
    };
    if (two)
      ksteps(std::true_type{});
    else
      ksteps(std::false_type{});
    if (!late) fold(sc, two);
#pragma unroll
    for (int c = 0; c < C32; ++c) scp[c] = sc[c];
    if ((kt & 1) == 1 || kt + 1 == KT) {
      if (late) fold(scp, two);  // the window's products go in before its correction
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        if (rt == 1 && !two) break;
#pragma unroll
        for (int c = 0; c < C32; ++c)
          acc[rt][c] = __builtin_amdgcn_mfma_f32_32x32x2f32(za[rt], zb[c], acc[rt][c], 0, 0, 0);
      }
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) za[rt] = 0.f;
#pragma unroll
      for (int c = 0; c < C32; ++c) zb[c] = 0.f;
    }
  };

  // ---- epilogue of item j: register i of tile (rt, c) = row mw*64 + 32*rt +
  // 8*(i/4) + 4*h + i%4 of column c32 of the tile ----
  auto row_of = [&](int rt, int i) { return mw * 64 + 32 * rt + 8 * (i >> 2) + 4 * h + (i & 3); };
  auto epilogue = [&](int j, const Plan& P) {
    const int* R = Rid[j % 3];
    if constexpr (EPI == EPI_SILU) {
      // h = silu(g) * u, rounded to the output type (hardware conversions,
      // round to nearest even).  Stores: lanes c32 and c32 ^ 1 swap one value
      // per row pair (DPP), so the even lane writes columns (c, c + 1) of the
      // even row and the odd lane those of the odd row, one 4-byte store each.
      float rs[32];
      const int64_t col2 = P.nb * WGN + nw * CTW * 16 + (c32 & ~1);
      const bool odd = (c32 & 1) != 0, bf = p.y_dtype == CCQ_BF16;
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          float hv[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float g = acc[rt][0][2 * m + e], u = acc[rt][1][2 * m + e];
            hv[e] = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
          }
          // own rounded values (rows 2m, 2m + 1 of this column) for the group sums
          uint32_t own;
          if (bf) {
            own = bf16x2_bits(hv[0], hv[1]);
            rs[rt * 16 + 2 * m] = __uint_as_float(own << 16);
            rs[rt * 16 + 2 * m + 1] = __uint_as_float(own & 0xFFFF0000u);
          } else {
            own = f32_to_f16_bits(hv[0]) | (f32_to_f16_bits(hv[1]) << 16);
            rs[rt * 16 + 2 * m] = f16_bits_to_f32(own & 0xFFFFu);
            rs[rt * 16 + 2 * m + 1] = f16_bits_to_f32(own >> 16);
          }
          // the even lane sends row 2m + 1, the odd lane row 2m
          const uint32_t send = odd ? (own & 0xFFFFu) : (own >> 16);
          const uint32_t recv = (uint32_t)__builtin_amdgcn_mov_dpp((int)send, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
          const uint32_t word = odd ? (recv | (own & 0xFFFF0000u)) : ((own & 0xFFFFu) | (recv << 16));
          const int row = row_of(rt, 2 * m + (odd ? 1 : 0));
          if (row < P.nvalid) *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(p.y) + (int64_t)R[row] * p.ldy + col2) = word;
          if (row_of(rt, 2 * m) >= P.nvalid) rs[rt * 16 + 2 * m] = 0.f;
          if (row_of(rt, 2 * m + 1) >= P.nvalid) rs[rt * 16 + 2 * m + 1] = 0.f;
        }
      if (p.sxo != nullptr) {
        // group sums of the stored rows over this item's 128 columns: 32 per
        // wave by butterfly, then the 4 column waves through LDS
        const float part_sum = half_wave_row_reduce<false>(rs, c32);
        part[nw * GG_BM + row_of(c32 >> 4, c32 & 15)] = part_sum;
        lds_barrier();
        if (tid < P.nvalid)
          p.sxo[(int64_t)R[tid] * p.ldsxo + P.nb] =
              ((part[tid] + part[GG_BM + tid]) + part[2 * GG_BM + tid]) + part[3 * GG_BM + tid];
      }
    } else {
      // rows of columns (c, c + 1) per store, as above: the even lane writes
      // the even row of a row pair, the odd lane the odd row
      const bool odd = (c32 & 1) != 0;
      const int64_t col2 = P.nb * WGN + nw * CTW * 16 + (c32 & ~1);
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          const int row = row_of(rt, 2 * m + (odd ? 1 : 0));
#pragma unroll
          for (int c = 0; c < C32; ++c) {
            const float v0 = acc[rt][c][2 * m], v1 = acc[rt][c][2 * m + 1];
            const float fs = odd ? v0 : v1;
            const float fr = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(fs), 0xB1, 0xF, 0xF, false));
            const float lo = odd ? fr : v0, hi = odd ? v1 : fr;  // columns (c & ~1), (c | 1) of the row
            if (row < P.nvalid) {
              const int64_t o = (int64_t)R[row] * p.ldy + col2 + c * 32;
              if (p.y_dtype == CCQ_F32)
                *reinterpret_cast<f32x2*>(reinterpret_cast<float*>(p.y) + o) = f32x2{lo, hi};
              else if (p.y_dtype == CCQ_BF16)
                *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(p.y) + o) = bf16x2_bits(lo, hi);
              else
                *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(p.y) + o) =
                    f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
            }
          }
        }
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int c = 0; c < C32; ++c) acc[rt][c] = f32x16{};
  };

  // ---- pipeline over all k-steps of all items of this workgroup: a ring of
  // 3 k-tiles, loads two k-steps ahead (across item boundaries) ----
  Plan cur, nxt;
  make_plan(0, cur);
  if (nmine > 1) make_plan(1, nxt);
  issue(cur, 0, 0);
  if (total > 1) issue(KT > 1 ? cur : nxt, KT > 1 ? 1 : 0, 1);
  // the ring slot is a run-time index: the ring lives in LDS only
  int j = 0, kt = 0, slot = 0;
  for (int g = 0; g < total; ++g) {
    if (g + 1 < total)
      wait_stage<7>(ncopy);
    else
      wait_vmcnt<0>();
    lds_barrier();
    if (kt == 0 && j + 2 < nmine) fetch_rows(j + 2);
    if (kt == KT - 2 && j + 1 < nmine) make_plan(j + 1, nxt);
    const bool last = kt + 1 == KT;
    const int slot2 = slot == 0 ? 2 : slot - 1;  // (slot + 2) % 3
    auto mid = [&]() {
      if (!last && g + 2 < total) issue(kt + 2 < KT ? cur : nxt, kt + 2 < KT ? kt + 2 : kt + 2 - KT, slot2);
    };
    if (mw * 64 < cur.nvalid)
      compute(slot, kt, mw * 64 + 32 < cur.nvalid, mid);
    else
      mid();
    if (last) {
      epilogue(j, cur);
      // the next item's second k-step is issued after the stores, so the
      // wait of the next k-step does not hold it back
      if (g + 2 < total) issue(nxt, 1, slot2);
      cur = nxt;
      ++j;
      kt = 0;
    } else {
      ++kt;
    }
    slot = slot == 2 ? 0 : slot + 1;
  }
}

// Sx[row][g] = sum of the 128 activations of group g of the row (float32,
// fixed order): 16 lanes per (row, group), 8 elements per lane.  With
// rows_out, also the row ids of a dense schedule: rows_out[i] = i < M ? i : -1
// for i < nrows_out.
template <typename AT>
__global__ __launch_bounds__(256) void row_group_sums_kernel(const AT* __restrict__ x, int64_t ldx, int64_t M,
                                                             int64_t KT, float* __restrict__ out, int64_t ldo,
                                                             int32_t* __restrict__ rows_out, int64_t nrows_out) {
  using V = typename Act<AT>::vec;
  const int64_t gt = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (rows_out != nullptr && gt < nrows_out) rows_out[gt] = gt < M ? (int32_t)gt : -1;
  const int64_t g = gt >> 4;
  const int part = threadIdx.x & 15;
  const bool ok = g < M * KT;
  const int64_t row = ok ? (int64_t)((uint32_t)g / (uint32_t)KT) : 0, kt = ok ? g - row * KT : 0;  // M * KT < 2^31
  float s = 0.f;
  if (ok) {
    const V v = *reinterpret_cast<const V*>(x + row * ldx + kt * 128 + part * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) s += (float)v[e];
  }
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) s += __shfl_xor(s, off, 64);
  if (ok && part == 0) out[row * ldo + kt] = s;
}

static int launch_row_group_sums(const void* x, int x_bf16, int64_t ldx, int64_t M, int64_t K, float* out,
                                 int64_t ldo, hipStream_t st, int32_t* rows_out = nullptr, int64_t nrows_out = 0) {
  const int64_t KT = K / 128, threads = M * KT * 16 > nrows_out ? M * KT * 16 : nrows_out;
  if (M * KT >= (1LL << 31)) return arg_error("row group sums: M=%lld x K/128=%lld too large", (long long)M, (long long)KT);
  const int64_t blocks = cdiv(threads, 256);
  if (x_bf16)
    launch(row_group_sums_kernel<__bf16>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const __bf16*)x, ldx, M, KT, out, ldo, rows_out, nrows_out);
  else
    launch(row_group_sums_kernel<_Float16>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const _Float16*)x, ldx, M, KT, out, ldo, rows_out, nrows_out);
  return launch_status("row group sums");
}

// Columns per workgroup of the grouped kernel for one matrix of N columns.
static int group_cols(int EPI, int64_t N) { return EPI == EPI_SILU ? 128 : (N % 256 == 0 ? 256 : 128); }

// Compute units of the current device (one persistent workgroup each).
static int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n < 8 ? 8 : n;  // the grouped kernel's schedule needs a workgroup on each of the 8 XCDs
  }
  return cus[dev];
}

template <typename AT, typename ST, int EPI>
static void launch_stream_t(const W4SP& p, int nq, dim3 grid, hipStream_t st) {
  const dim3 block(512);
  const bool mt4 = p.KT > 16;
  if constexpr (EPI == EPI_SILU) {
    if (p.logits != nullptr)  // routing inside the workgroups
      launch((w4_stream_kernel<AT, ST, EPI, 2, 2, true>), grid, block, 0, st, p);
    else
      launch((w4_stream_kernel<AT, ST, EPI, 2, 2>), grid, block, 0, st, p);
  } else if (nq == 2) {  // two quads: K <= 2048, two k-tiles per wave
    if constexpr (EPI == EPI_ROWS) {
      if (p.KT <= 8) {  // K <= 1024: one k-tile per wave, four jobs in flight
        launch((w4_stream_kernel<AT, ST, EPI, 1, 2>), grid, block, 0, st, p);
        return;
      }
    }
    launch((w4_stream_kernel<AT, ST, EPI, 2, 2>), grid, block, 0, st, p);
  } else if constexpr (EPI != EPI_SILU) {
    if (mt4)
      launch((w4_stream_kernel<AT, ST, EPI, 4, 1>), grid, block, 0, st, p);
    else
      launch((w4_stream_kernel<AT, ST, EPI, 2, 1>), grid, block, 0, st, p);
  }
}

template <int EPI>
static int launch_stream(const W4SP& p, int nq, int x_bf16, int s_bf16, int64_t tiles, hipStream_t st) {
  if (p.KT > 16 && (tiles != 1 || p.meta != nullptr)) return arg_error("w4 stream gemm: K > 2048 needs a single row tile");
  // the kernel splits a schedule's jobs over the workgroups in 32-bit arithmetic
  if ((p.meta != nullptr || p.logits != nullptr) && tiles * (p.N / 16) >= (1 << 23))
    return arg_error("w4 stream gemm: %lld tiles x N=%d is too large a schedule", (long long)tiles, p.N);
  const int64_t jobs = tiles * (p.N / (EPI == EPI_SILU ? 16 : 16 * nq)), cus = device_cus();
  const dim3 grid((unsigned)(jobs < cus ? jobs : cus));
  if (x_bf16) {
    if (s_bf16)
      launch_stream_t<__bf16, __bf16, EPI>(p, nq, grid, st);
    else
      launch_stream_t<__bf16, _Float16, EPI>(p, nq, grid, st);
  } else {
    if (s_bf16)
      launch_stream_t<_Float16, __bf16, EPI>(p, nq, grid, st);
    else
      launch_stream_t<_Float16, _Float16, EPI>(p, nq, grid, st);
  }
  return launch_status("w4 stream gemm");
}

// tiles = schedule tiles the grid is sized for (the kernel reads the actual
// number from meta); one persistent workgroup per compute unit at most.
template <int EPI>
static int launch_group_gemm(const W4GP& p, int x_bf16, int s_bf16, int64_t tiles, hipStream_t st) {
  const int wgn = group_cols(EPI, p.N);
  const int64_t items = tiles * (p.N / wgn), cus = device_cus();
  const dim3 grid((unsigned)(items < cus ? items : cus)), block(512);
#define CCQ_LAUNCH_GG(AT, ST)                                                                  \
  do {                                                                                         \
    if (wgn == 256)                                                                            \
      launch((w4_group_gemm_kernel<AT, ST, EPI, (EPI == EPI_SILU ? 2 : 4)>), grid, \
                         block, 0, st, p);                                                     \
    else                                                                                       \
      launch((w4_group_gemm_kernel<AT, ST, EPI, 2>), grid, block, 0, st, p);      \
  } while (0)
  if (x_bf16) {
    if (s_bf16)
      CCQ_LAUNCH_GG(__bf16, __bf16);
    else
      CCQ_LAUNCH_GG(__bf16, _Float16);
  } else {
    if (s_bf16)
      CCQ_LAUNCH_GG(_Float16, __bf16);
    else
      CCQ_LAUNCH_GG(_Float16, _Float16);
  }
#undef CCQ_LAUNCH_GG
  return launch_status("w4 grouped gemm");
}

// The grouped kernel replaces the 16-row decode kernel once the average
// expert receives at least 16 rows (and the shape suits it: group 128,
// N a multiple of 128, and at least 2 k-tiles on both matrices, as hidden
// and inter are each the N of one matrix and the K of the other).
static bool use_group_gemm(int64_t n, int64_t E, int64_t G, int64_t N1, int64_t N2) {
  return n >= 16 * E && G == 128 && N1 % 128 == 0 && N2 % 128 == 0 && N1 >= 256 && N2 >= 256;
}


}  // namespace ccq

using namespace ccq;

static int grid1d(int64_t n) {
  int64_t g = cdiv(n, 256);
  return (int)(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

extern "C" int ccq_awq_dequant(const int32_t* qweight, const int32_t* qzeros, const void* scales, int scale_dtype,
                               float* out, int64_t K, int64_t N, int64_t group_size, void* stream) {
  CCQ_REQUIRE(K >= 0 && N >= 0, "ccq_awq_dequant: negative shape");
  CCQ_REQUIRE(N % 8 == 0, "ccq_awq_dequant: N=%lld not a multiple of 8", (long long)N);
  CCQ_REQUIRE(group_size > 0 && K % group_size == 0, "ccq_awq_dequant: K=%lld not a multiple of group %lld",
              (long long)K, (long long)group_size);
  CCQ_REQUIRE(scale_dtype == CCQ_F16 || scale_dtype == CCQ_BF16, "ccq_awq_dequant: scale_dtype must be f16|bf16");
  if (K == 0 || N == 0) return 0;
  CCQ_REQUIRE(qweight && qzeros && scales && out, "ccq_awq_dequant: null pointer");
  launch(awq_dequant_kernel, dim3(grid1d(K * N / 8)), dim3(256), 0, as_stream(stream),
                     (const uint32_t*)qweight, (const uint32_t*)qzeros, (const uint16_t*)scales,
                     scale_dtype == CCQ_BF16 ? 1 : 0, out, K, N, group_size);
  return launch_status("ccq_awq_dequant");
}

extern "C" int ccq_awq_repack(const int32_t* qweight, int32_t* tiled, int64_t K, int64_t N, void* stream) {
  CCQ_REQUIRE(K >= 0 && N >= 0, "ccq_awq_repack: negative shape");
  CCQ_REQUIRE(K % 128 == 0 && N % 16 == 0, "ccq_awq_repack: need K %% 128 == 0 and N %% 16 == 0 (K=%lld N=%lld)",
              (long long)K, (long long)N);
  if (K == 0 || N == 0) return 0;
  CCQ_REQUIRE(qweight && tiled, "ccq_awq_repack: null pointer");
  CCQ_REQUIRE((const void*)qweight != (const void*)tiled, "ccq_awq_repack: in-place repack is not supported");
  launch(awq_repack_kernel, dim3(grid1d(K * N / 8)), dim3(256), 0, as_stream(stream),
                     (const uint32_t*)qweight, (uint32_t*)tiled, K, N);
  return launch_status("ccq_awq_repack");
}

extern "C" int ccq_awq_unpack_tiled(const int32_t* tiled, int32_t* qweight, int64_t K, int64_t N, void* stream) {
  CCQ_REQUIRE(K >= 0 && N >= 0, "ccq_awq_unpack_tiled: negative shape");
  CCQ_REQUIRE(K % 128 == 0 && N % 16 == 0, "ccq_awq_unpack_tiled: need K %% 128 == 0 and N %% 16 == 0");
  if (K == 0 || N == 0) return 0;
  CCQ_REQUIRE(qweight && tiled, "ccq_awq_unpack_tiled: null pointer");
  CCQ_REQUIRE((const void*)qweight != (const void*)tiled, "ccq_awq_unpack_tiled: in-place is not supported");
  launch(awq_unpack_tiled_kernel, dim3(grid1d(K * N / 8)), dim3(256), 0, as_stream(stream),
                     (const uint32_t*)tiled, (uint32_t*)qweight, K, N);
  return launch_status("ccq_awq_unpack_tiled");
}

extern "C" int64_t ccq_awq_sz_words(int64_t K, int64_t group_size) {
  if (K <= 0 || K % 128 || !valid_group(group_size)) return 0;
  return sz_words_per_column(K, group_size);
}

extern "C" int ccq_awq_pack_sz(const int32_t* qzeros, const void* scales, int scale_dtype, uint32_t* sz, int64_t K,
                               int64_t N, int64_t group_size, void* stream) {
  CCQ_REQUIRE(K >= 0 && N >= 0, "ccq_awq_pack_sz: negative shape");
  CCQ_REQUIRE(K % 128 == 0 && N % 16 == 0, "ccq_awq_pack_sz: need K %% 128 == 0 and N %% 16 == 0 (K=%lld N=%lld)",
              (long long)K, (long long)N);
  CCQ_REQUIRE(valid_group(group_size), "ccq_awq_pack_sz: group_size=%lld not in {32, 64, 128}", (long long)group_size);
  CCQ_REQUIRE(scale_dtype == CCQ_F16 || scale_dtype == CCQ_BF16, "ccq_awq_pack_sz: scale_dtype must be f16|bf16");
  if (K == 0 || N == 0) return 0;
  CCQ_REQUIRE(qzeros && scales && sz, "ccq_awq_pack_sz: null pointer");
  launch(awq_pack_sz_kernel, dim3(grid1d(N * sz_words_per_column(K, group_size))), dim3(256), 0,
                     as_stream(stream), (const uint32_t*)qzeros, (const uint16_t*)scales, sz, K, N, group_size);
  return launch_status("ccq_awq_pack_sz");
}

namespace {
// The dense GEMM switches to the grouped kernel for prefill-sized M.
bool gemm_grouped(int64_t M, int64_t K, int64_t N, int64_t G) {
  return M > 64 && G == 128 && N % 128 == 0 && K >= 256;
}
}  // namespace

extern "C" size_t ccq_w4_gemm_workspace_size(int64_t M, int64_t K, int64_t N, int64_t group_size) {
  if (M <= 0 || K <= 0 || K % 128 || !gemm_grouped(M, K, N, group_size)) return 0;
  // row group sums, then the row ids of the 128-row tiles
  return align256((size_t)M * (size_t)(K / 128) * 4) + align256((size_t)cdiv(M, GG_BM) * GG_BM * 4);
}

extern "C" int ccq_w4_gemm(const void* x, int x_dtype, const int32_t* w_tiled, const uint32_t* sz, int scale_dtype,
                           void* y, int y_dtype, int64_t M, int64_t K, int64_t N, int64_t group_size,
                           void* workspace, size_t workspace_bytes, void* stream) {
  CCQ_REQUIRE(M >= 0 && K >= 0 && N >= 0, "ccq_w4_gemm: negative shape");
  CCQ_REQUIRE(K % 128 == 0 && N % 16 == 0, "ccq_w4_gemm: need K %% 128 == 0 and N %% 16 == 0 (K=%lld N=%lld)",
              (long long)K, (long long)N);
  CCQ_REQUIRE(valid_group(group_size), "ccq_w4_gemm: group_size=%lld not in {32, 64, 128}", (long long)group_size);
  CCQ_REQUIRE(x_dtype == CCQ_F16 || x_dtype == CCQ_BF16, "ccq_w4_gemm: x_dtype must be f16|bf16");
  CCQ_REQUIRE(scale_dtype == CCQ_F16 || scale_dtype == CCQ_BF16, "ccq_w4_gemm: scale_dtype must be f16|bf16");
  CCQ_REQUIRE(y_dtype == CCQ_F16 || y_dtype == CCQ_BF16 || y_dtype == CCQ_F32, "ccq_w4_gemm: bad y_dtype");
  CCQ_REQUIRE(K <= (1 << 20) && N / 16 <= 0x7fffffff, "ccq_w4_gemm: K=%lld or N=%lld too large", (long long)K,
              (long long)N);
  const bool grouped = gemm_grouped(M, K, N, group_size);
  CCQ_REQUIRE(grouped || cdiv(M, 16) <= 65535, "ccq_w4_gemm: M=%lld too large", (long long)M);
  if (M == 0 || N == 0) return 0;
  CCQ_REQUIRE(K > 0, "ccq_w4_gemm: K == 0");
  CCQ_REQUIRE(x && w_tiled && sz && y, "ccq_w4_gemm: null pointer");
  CCQ_REQUIRE(aligned(x, 16) && aligned(w_tiled, 16) && aligned(sz, 16),
              "ccq_w4_gemm: x, w_tiled and sz must be 16-byte aligned");
  if (grouped) {
    // prefill-sized: 128-row tiles stream the weight once per tile
    const size_t need = ccq_w4_gemm_workspace_size(M, K, N, group_size);
    CCQ_REQUIRE(workspace && workspace_bytes >= need && aligned(workspace, 256),
                "ccq_w4_gemm: workspace of %zu bytes (256-byte aligned) needed for M=%lld, %zu given", need,
                (long long)M, workspace_bytes);
    CCQ_REQUIRE(M * K * 2 < (int64_t)1 << 32, "ccq_w4_gemm: activations of %lld x %lld exceed 4 GiB",
                (long long)M, (long long)K);
    CCQ_REQUIRE(cdiv(M, GG_BM) * (N / 128) <= 0x7fffffff, "ccq_w4_gemm: M=%lld too large", (long long)M);
    hipStream_t st = as_stream(stream);
    float* sx = (float*)workspace;
    int32_t* rows = (int32_t*)((char*)workspace + align256((size_t)M * (size_t)(K / 128) * 4));
    const int64_t tiles = cdiv(M, GG_BM);
    int rc = launch_row_group_sums(x, x_dtype == CCQ_BF16, K, M, K, sx, K / 128, st, rows, tiles * GG_BM);
    if (rc) return rc;
    W4GP g = {};
    g.x = x;
    g.ldx = K;
    g.sx = sx;
    g.ldsx = K / 128;
    g.rows = rows;
    g.row_div = 1;
    g.tiles = (int)cdiv(M, GG_BM);
    g.w0 = (const uint32_t*)w_tiled;
    g.sz0 = sz;
    g.y = y;
    g.ldy = N;
    g.y_dtype = y_dtype;
    g.M = (int)M;
    g.N = (int)N;
    g.K = (int)K;
    g.KT = (int)(K / 128);
    g.szw = (int)sz_words_per_column(K, group_size);
    g.nib_mask = 0x000F000Fu;
    return launch_group_gemm<EPI_STORE>(g, x_dtype == CCQ_BF16, scale_dtype == CCQ_BF16, g.tiles, st);
  }
  const int64_t szw_d = sz_words_per_column(K, group_size);
  // 16-column jobs (one quad) when 32-column jobs would leave CUs idle
  // (K=2048 N=5632: 176 jobs of 32 columns, 352 of 16)
  int nq = stream_nq(EPI_STORE, N, K, group_size);
  if (nq == 2 && N / 32 < device_cus() && K <= 4096) nq = 1;
  if (M <= 16 && nq > 0) {
    // decode: one 16-row tile, weights streamed once
    W4SP w = {};
    w.x = x;
    w.ldx = K;
    w.row_div = 1;
    w.tiles = 1;
    w.w0 = (const uint32_t*)w_tiled;
    w.sz0 = sz;
    w.y = y;
    w.ldy = N;
    w.y_dtype = y_dtype;
    w.M = (int)M;
    w.N = (int)N;
    w.K = (int)K;
    w.KT = (int)(K / 128);
    w.szw = (int)szw_d;
    w.nib_mask = 0x000F000Fu;
    return launch_stream<EPI_STORE>(w, nq, x_dtype == CCQ_BF16, scale_dtype == CCQ_BF16, 1, as_stream(stream));
  }
  const int64_t tiles = cdiv(M, 16);
  const SkinnyPlan pl = plan_skinny(K, N, group_size, 1, gemm_nb(M));
  SkinnyP p = {};
  p.x = x;
  p.ldx = K;
  p.row_div = 1;
  p.w0 = (const uint32_t*)w_tiled;
  p.sz0 = sz;
  p.y = y;
  p.ldy = N;
  p.y_dtype = y_dtype;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.KT = (int)(K / 128);
  p.szw = (int)sz_words_per_column(K, group_size);
  launch_skinny<EPI_STORE>(p, x_dtype == CCQ_BF16, scale_dtype == CCQ_BF16, pl, tiles, as_stream(stream),
                           (int)group_size);
  return launch_status("ccq_w4_gemm");
}

// ------------------------------------------------------------ MoE W4 FFN --
namespace {

int check_experts(const ccq_w4_experts* ex, const char* name) {
  CCQ_REQUIRE(ex != nullptr, "%s: null expert descriptor", name);
  CCQ_REQUIRE(ex->num_experts >= 1 && ex->num_experts <= 1024, "%s: num_experts=%lld outside [1, 1024]", name,
              (long long)ex->num_experts);
  CCQ_REQUIRE(ex->hidden > 0 && ex->inter > 0 && ex->hidden % 128 == 0 && ex->inter % 128 == 0,
              "%s: hidden=%lld and inter=%lld must be positive multiples of 128", name, (long long)ex->hidden,
              (long long)ex->inter);
  CCQ_REQUIRE(ex->hidden <= (1 << 20) && ex->inter <= (1 << 20), "%s: hidden/inter too large", name);
  CCQ_REQUIRE(valid_group(ex->group_size), "%s: group_size=%lld not in {32, 64, 128}", name,
              (long long)ex->group_size);
  CCQ_REQUIRE(ex->scale_dtype == CCQ_F16 || ex->scale_dtype == CCQ_BF16, "%s: scale_dtype must be f16|bf16", name);
  return 0;
}

int check_expert_ptrs(const ccq_w4_experts* ex, bool gate_up, const char* name) {
  if (gate_up) {
    CCQ_REQUIRE(ex->w_gate && ex->sz_gate && ex->w_up && ex->sz_up, "%s: null gate/up weight pointer", name);
    CCQ_REQUIRE(aligned(ex->w_gate, 16) && aligned(ex->w_up, 16) && aligned(ex->sz_gate, 16) &&
                    aligned(ex->sz_up, 16),
                "%s: tiled weights and sz must be 16-byte aligned", name);
  } else {
    CCQ_REQUIRE(ex->w_down && ex->sz_down, "%s: null down weight pointer", name);
    CCQ_REQUIRE(aligned(ex->w_down, 16) && aligned(ex->sz_down, 16),
                "%s: tiled weights and sz must be 16-byte aligned", name);
  }
  return 0;
}

// Workspace of ccq_moe_w4_ffn: the schedule, the SiLU(gate)*up intermediate
// and the per-assignment down rows.
struct MoeLayout {
  int64_t n, max_tiles;
  int tile_m;       // rows per schedule tile: 16 (decode kernel) or 128 (grouped kernel)
  bool grouped;
  size_t off_sorted, off_tile_expert, off_meta, off_counts, off_inter, off_rows, off_sx, off_sxh, off_ids, off_wts,
      off_align, total;
};

MoeLayout moe_layout(int64_t T, int64_t k, const ccq_w4_experts* ex, int x_bytes) {
  MoeLayout L;
  L.n = T * k;
  L.grouped = use_group_gemm(L.n, ex->num_experts, ex->group_size, ex->inter, ex->hidden);
  L.tile_m = L.grouped ? GG_BM : 16;
  L.max_tiles = ccq_moe_align_max_tiles(L.n, ex->num_experts, L.tile_m);
  size_t o = 0;
  L.off_sorted = o;
  o += align256((size_t)L.max_tiles * L.tile_m * 4);
  L.off_tile_expert = o;
  o += align256((size_t)L.max_tiles * 4);
  L.off_meta = o;
  o += 256;
  L.off_counts = o;
  o += align256((size_t)ex->num_experts * 4);
  L.off_inter = o;
  o += align256((size_t)L.n * ex->inter * x_bytes);
  L.off_rows = o;
  o += align256((size_t)L.n * ex->hidden * 4);
  L.off_sx = o;   // grouped: group sums of x rows and of the intermediate rows
  L.off_sxh = o;
  if (L.grouped) {
    o += align256((size_t)T * (ex->hidden / 128) * 4);
    L.off_sxh = o;
    o += align256((size_t)L.n * (ex->inter / 128) * 4);
  }
  L.off_ids = o;  // routing of ccq_moe_w4_forward when the caller keeps none
  o += align256((size_t)L.n * 8);
  L.off_wts = o;
  o += align256((size_t)L.n * 4);
  L.off_align = o;  // per-chunk tables of the schedule of large batches
  o += align256(align_scratch_bytes(L.n, ex->num_experts));
  L.total = o;
  return L;
}

// The streaming kernel's parameters for a decode stage set up as SkinnyP.
W4SP stream_params(const SkinnyP& p) {
  W4SP w = {};
  w.x = p.x;
  w.ldx = p.ldx;
  w.rows = p.rows;
  w.row_div = p.row_div;
  w.tile_expert = p.tile_expert;
  w.meta = p.meta;
  w.w0 = p.w0;
  w.sz0 = p.sz0;
  w.w1 = p.w1;
  w.sz1 = p.sz1;
  w.w_es = p.w_es;
  w.sz_es = p.sz_es;
  w.y = p.y;
  w.ldy = p.ldy;
  w.y_dtype = p.y_dtype;
  w.M = p.M;
  w.N = p.N;
  w.K = p.K;
  w.KT = p.KT;
  w.szw = p.szw;
  w.nib_mask = 0x000F000Fu;
  return w;
}

SkinnyP grouped_params(const int32_t* sorted_ids, const int32_t* tile_expert, const int32_t* meta,
                       const ccq_w4_experts* ex) {
  SkinnyP p = {};
  p.rows = sorted_ids;
  p.tile_expert = tile_expert;
  p.meta = meta;
  return p;
}

int run_gate_up(const void* x, int x_dtype, int64_t k, const int32_t* sorted_ids, const int32_t* tile_expert,
                const int32_t* meta, int64_t max_tiles, void* inter, const ccq_w4_experts* ex, hipStream_t st) {
  const int64_t H = ex->hidden, I = ex->inter, G = ex->group_size;
  SkinnyP p = grouped_params(sorted_ids, tile_expert, meta, ex);
  p.x = x;
  p.ldx = H;
  p.row_div = (int)k;
  p.w0 = (const uint32_t*)ex->w_gate;
  p.sz0 = ex->sz_gate;
  p.w1 = (const uint32_t*)ex->w_up;
  p.sz1 = ex->sz_up;
  p.szw = (int)sz_words_per_column(H, G);
  p.w_es = H * I / 8;
  p.sz_es = I * p.szw;
  p.y = inter;
  p.ldy = I;
  p.y_dtype = x_dtype;
  p.N = (int)I;
  p.K = (int)H;
  p.KT = (int)(H / 128);
  const int nq = stream_nq(EPI_SILU, I, H, G);
  if (nq > 0 && max_tiles <= device_cus()) {
    const W4SP w = stream_params(p);
    return launch_stream<EPI_SILU>(w, nq, x_dtype == CCQ_BF16, ex->scale_dtype == CCQ_BF16, max_tiles, st);
  }
  const SkinnyPlan pl = plan_skinny(H, I, G, 2, 1);
  launch_skinny<EPI_SILU>(p, x_dtype == CCQ_BF16, ex->scale_dtype == CCQ_BF16, pl, max_tiles, st, (int)G);
  return launch_status("moe_w4 gate_up");
}

int run_down(const void* inter, int x_dtype, const int32_t* sorted_ids, const int32_t* tile_expert,
             const int32_t* meta, int64_t max_tiles, float* rows, const ccq_w4_experts* ex, hipStream_t st) {
  const int64_t H = ex->hidden, I = ex->inter, G = ex->group_size;
  SkinnyP d = grouped_params(sorted_ids, tile_expert, meta, ex);
  d.x = inter;
  d.ldx = I;
  d.row_div = 1;
  d.w0 = (const uint32_t*)ex->w_down;
  d.sz0 = ex->sz_down;
  d.szw = (int)sz_words_per_column(I, G);
  d.w_es = I * H / 8;
  d.sz_es = H * d.szw;
  d.y = rows;
  d.ldy = H;
  d.y_dtype = CCQ_F32;
  d.N = (int)H;
  d.K = (int)I;
  d.KT = (int)(I / 128);
  const int nq = stream_nq(EPI_ROWS, H, I, G);
  if (nq > 0 && max_tiles <= device_cus()) {
    const W4SP w = stream_params(d);
    return launch_stream<EPI_ROWS>(w, nq, x_dtype == CCQ_BF16, ex->scale_dtype == CCQ_BF16, max_tiles, st);
  }
  const SkinnyPlan pl = plan_skinny(I, H, G, 1, 1);
  launch_skinny<EPI_ROWS>(d, x_dtype == CCQ_BF16, ex->scale_dtype == CCQ_BF16, pl, max_tiles, st, (int)G);
  return launch_status("moe_w4 down");
}

int check_stage_args(const void* a, int x_dtype, const int32_t* sorted_ids, const int32_t* tile_expert,
                     const int32_t* meta, int64_t max_tiles, const void* out, const ccq_w4_experts* ex,
                     bool gate_up, const char* name) {
  int rc = check_experts(ex, name);
  if (rc) return rc;
  rc = check_expert_ptrs(ex, gate_up, name);
  if (rc) return rc;
  CCQ_REQUIRE(x_dtype == CCQ_F16 || x_dtype == CCQ_BF16, "%s: activation dtype must be f16|bf16", name);
  CCQ_REQUIRE(max_tiles >= 1 && max_tiles <= 65535, "%s: max_tiles=%lld outside [1, 65535]", name,
              (long long)max_tiles);
  CCQ_REQUIRE(a && sorted_ids && tile_expert && meta && out, "%s: null pointer", name);
  CCQ_REQUIRE(aligned(a, 16), "%s: activations must be 16-byte aligned", name);
  return 0;
}

}  // namespace

extern "C" int ccq_moe_w4_gate_up(const void* x, int x_dtype, int64_t k, const int32_t* sorted_ids,
                                  const int32_t* tile_expert, const int32_t* meta, int64_t max_tiles, void* inter,
                                  const ccq_w4_experts* ex, void* stream) {
  int rc = check_stage_args(x, x_dtype, sorted_ids, tile_expert, meta, max_tiles, inter, ex, true,
                            "ccq_moe_w4_gate_up");
  if (rc) return rc;
  CCQ_REQUIRE(k >= 1 && k <= ex->num_experts, "ccq_moe_w4_gate_up: k=%lld outside [1, E]", (long long)k);
  return run_gate_up(x, x_dtype, k, sorted_ids, tile_expert, meta, max_tiles, inter, ex, as_stream(stream));
}

extern "C" int ccq_moe_w4_down(const void* inter, int x_dtype, const int32_t* sorted_ids, const int32_t* tile_expert,
                               const int32_t* meta, int64_t max_tiles, float* rows, const ccq_w4_experts* ex,
                               void* stream) {
  int rc = check_stage_args(inter, x_dtype, sorted_ids, tile_expert, meta, max_tiles, rows, ex, false,
                            "ccq_moe_w4_down");
  if (rc) return rc;
  return run_down(inter, x_dtype, sorted_ids, tile_expert, meta, max_tiles, rows, ex, as_stream(stream));
}

extern "C" size_t ccq_moe_w4_workspace_size(int64_t T, int64_t k, const ccq_w4_experts* ex) {
  if (T <= 0 || k <= 0 || check_experts(ex, "ccq_moe_w4_workspace_size") != 0) return 0;
  return moe_layout(T, k, ex, 2).total;
}

static int moe_w4_ffn(const void* x, int x_dtype, const int64_t* ids, const float* weights, void* y, int y_dtype,
                      int64_t T, int64_t k, const ccq_w4_experts* ex, void* workspace, size_t workspace_bytes,
                      void* stream, const float* shared, float shared_gate);

extern "C" int ccq_moe_w4_ffn(const void* x, int x_dtype, const int64_t* ids, const float* weights, void* y,
                              int y_dtype, int64_t T, int64_t k, const ccq_w4_experts* ex, void* workspace,
                              size_t workspace_bytes, void* stream) {
  return moe_w4_ffn(x, x_dtype, ids, weights, y, y_dtype, T, k, ex, workspace, workspace_bytes, stream, nullptr, 0.f);
}

extern "C" int ccq_moe_w4_ffn_shared(const void* x, int x_dtype, const int64_t* ids, const float* weights,
                                     const float* shared, float shared_gate, void* y, int y_dtype, int64_t T,
                                     int64_t k, const ccq_w4_experts* ex, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  CCQ_REQUIRE(shared || T == 0, "ccq_moe_w4_ffn_shared: null shared");
  return moe_w4_ffn(x, x_dtype, ids, weights, y, y_dtype, T, k, ex, workspace, workspace_bytes, stream, shared,
                    shared_gate);
}

static int moe_w4_ffn(const void* x, int x_dtype, const int64_t* ids, const float* weights, void* y, int y_dtype,
                      int64_t T, int64_t k, const ccq_w4_experts* ex, void* workspace, size_t workspace_bytes,
                      void* stream, const float* shared, float shared_gate) {
  int rc = check_experts(ex, "ccq_moe_w4_ffn");
  if (rc) return rc;
  CCQ_REQUIRE(T >= 0 && k >= 1 && k <= ex->num_experts, "ccq_moe_w4_ffn: bad T=%lld / k=%lld", (long long)T,
              (long long)k);
  CCQ_REQUIRE(T * k <= 65536, "ccq_moe_w4_ffn: T*k=%lld > 65536", (long long)(T * k));
  CCQ_REQUIRE(x_dtype == CCQ_F16 || x_dtype == CCQ_BF16, "ccq_moe_w4_ffn: x_dtype must be f16|bf16");
  CCQ_REQUIRE(y_dtype == CCQ_F16 || y_dtype == CCQ_BF16 || y_dtype == CCQ_F32, "ccq_moe_w4_ffn: bad y_dtype");
  CCQ_REQUIRE(T <= 65535, "ccq_moe_w4_ffn: T=%lld > 65535", (long long)T);
  if (T == 0) return 0;
  CCQ_REQUIRE(x && ids && weights && y, "ccq_moe_w4_ffn: null pointer");
  rc = check_expert_ptrs(ex, true, "ccq_moe_w4_ffn");
  if (rc) return rc;
  rc = check_expert_ptrs(ex, false, "ccq_moe_w4_ffn");
  if (rc) return rc;
  CCQ_REQUIRE(aligned(x, 16), "ccq_moe_w4_ffn: x must be 16-byte aligned");
  const MoeLayout L = moe_layout(T, k, ex, 2);
  CCQ_REQUIRE(workspace && workspace_bytes >= L.total && aligned(workspace, 256),
              "ccq_moe_w4_ffn: workspace of %zu bytes (256-byte aligned) needed, %zu given", L.total,
              workspace_bytes);
  hipStream_t st = as_stream(stream);
  char* ws = (char*)workspace;
  int32_t* sorted = (int32_t*)(ws + L.off_sorted);
  int32_t* tile_expert = (int32_t*)(ws + L.off_tile_expert);
  int32_t* meta = (int32_t*)(ws + L.off_meta);
  int32_t* counts = (int32_t*)(ws + L.off_counts);
  void* inter = ws + L.off_inter;
  float* rows = (float*)(ws + L.off_rows);

  CCQ_REQUIRE(L.max_tiles * 2 <= 65535, "ccq_moe_w4_ffn: too many tiles");
  if (L.grouped) {
    const int64_t H = ex->hidden, I = ex->inter, G = ex->group_size;
    CCQ_REQUIRE(T * H * 2 < (int64_t)1 << 32 && L.n * I * 2 < (int64_t)1 << 32,
                "ccq_moe_w4_ffn: activations exceed 4 GiB");
    float* sx = (float*)(ws + L.off_sx);
    float* sxh = (float*)(ws + L.off_sxh);
    // the layer input's row group sums, in the schedule's launch where it is
    // the one-workgroup kernel
    bool sums_done = false;
    const AlignSide side = {ALIGN_SIDE_SUMS, x, x_dtype, H, T, H / 128, sx, H / 128};
    rc = launch_align_side(ids, L.n, ex->num_experts, L.tile_m, sorted, tile_expert, meta, counts, st,
                           ws + L.off_align, L.total - L.off_align, side, sums_done);
    if (rc) return rc;
    if (!sums_done) rc = launch_row_group_sums(x, x_dtype == CCQ_BF16, H, T, H, sx, H / 128, st);
    if (rc) return rc;
    W4GP g = {};
    g.x = x;
    g.ldx = H;
    g.sx = sx;
    g.ldsx = H / 128;
    g.rows = sorted;
    g.row_div = (int)k;
    g.tile_expert = tile_expert;
    g.meta = meta;
    g.w0 = (const uint32_t*)ex->w_gate;
    g.sz0 = ex->sz_gate;
    g.w1 = (const uint32_t*)ex->w_up;
    g.sz1 = ex->sz_up;
    g.szw = (int)sz_words_per_column(H, G);
    g.w_es = H * I / 8;
    g.sz_es = I * g.szw;
    g.y = inter;
    g.ldy = I;
    g.y_dtype = x_dtype;
    g.sxo = sxh;
    g.ldsxo = I / 128;
    g.N = (int)I;
    g.K = (int)H;
    g.KT = (int)(H / 128);
    g.nib_mask = 0x000F000Fu;
    rc = launch_group_gemm<EPI_SILU>(g, x_dtype == CCQ_BF16, ex->scale_dtype == CCQ_BF16, L.max_tiles, st);
    if (rc) return rc;
    W4GP d = {};
    d.x = inter;
    d.ldx = I;
    d.sx = sxh;
    d.ldsx = I / 128;
    d.rows = sorted;
    d.row_div = 1;
    d.tile_expert = tile_expert;
    d.meta = meta;
    d.w0 = (const uint32_t*)ex->w_down;
    d.sz0 = ex->sz_down;
    d.szw = (int)sz_words_per_column(I, G);
    d.w_es = I * H / 8;
    d.sz_es = H * d.szw;
    d.y = rows;
    d.ldy = H;
    d.y_dtype = CCQ_BF16;
    d.N = (int)H;
    d.K = (int)I;
    d.KT = (int)(I / 128);
    d.nib_mask = 0x000F000Fu;
    rc = launch_group_gemm<EPI_ROWS>(d, x_dtype == CCQ_BF16, ex->scale_dtype == CCQ_BF16, L.max_tiles, st);
    if (rc) return rc;
  } else {
    rc = launch_align(ids, L.n, ex->num_experts, L.tile_m, sorted, tile_expert, meta, counts, st,
                      ws + L.off_align, L.total - L.off_align);
    if (rc) return rc;
    rc = run_gate_up(x, x_dtype, k, sorted, tile_expert, meta, L.max_tiles, inter, ex, st);
    if (rc) return rc;
    rc = run_down(inter, x_dtype, sorted, tile_expert, meta, L.max_tiles, rows, ex, st);
    if (rc) return rc;
  }
  // the grouped path stores the down rows as bf16 (half the traffic of the
  // row write and of the combine's read)
  return launch_combine(rows, L.grouped ? CCQ_BF16 : CCQ_F32, weights, ids, ex->num_experts, y, y_dtype, T, k,
                        ex->hidden, st, shared, shared_gate);
}

// Whether a decode batch routes inside the gate/up kernel: the streaming
// kernels take both stages, the batch fits the in-workgroup router and has
// at most 16 tokens (the gate/up kernel's MFMA rows are the tokens).
static bool fused_route(const MoeLayout& L, const ccq_w4_experts* ex, int64_t k) {
  const int64_t H = ex->hidden, I = ex->inter, G = ex->group_size;
  return !L.grouped && L.n <= RT_MAXN && L.n / k <= 16 && ex->num_experts <= RT_MAXE && k <= 16 &&
         L.n / k * ex->num_experts <= RT_MAXLG &&
         stream_nq(EPI_SILU, I, H, G) > 0 && stream_nq(EPI_ROWS, H, I, G) > 0 && L.max_tiles <= device_cus() &&
         L.max_tiles <= RT_MAXTILES;
}

// Argument checks shared by ccq_moe_w4_forward and its routed gate/up stage
// (y is not used by the stage).
static int check_forward_args(const char* name, const void* x, int x_dtype, const float* logits, int64_t T,
                              int64_t k, int mode, const void* y, int y_dtype, const ccq_w4_experts* ex,
                              void* workspace, size_t workspace_bytes, bool need_y) {
  int rc = check_experts(ex, name);
  if (rc) return rc;
  CCQ_REQUIRE(T >= 0 && k >= 1 && k <= 16 && k <= ex->num_experts, "%s: bad T=%lld / k=%lld", name, (long long)T,
              (long long)k);
  CCQ_REQUIRE(mode >= 0 && mode <= 4, "%s: mode=%d not in {0,1,2,3,4}", name, mode);
  CCQ_REQUIRE(T * k <= 65536 && T <= 65535, "%s: T=%lld too large", name, (long long)T);
  CCQ_REQUIRE(x_dtype == CCQ_F16 || x_dtype == CCQ_BF16, "%s: x_dtype must be f16|bf16", name);
  CCQ_REQUIRE(!need_y || y_dtype == CCQ_F16 || y_dtype == CCQ_BF16 || y_dtype == CCQ_F32, "%s: bad y_dtype", name);
  if (T == 0) return 0;
  CCQ_REQUIRE(x && logits && (y || !need_y), "%s: null pointer", name);
  rc = check_expert_ptrs(ex, true, name);
  if (rc) return rc;
  rc = check_expert_ptrs(ex, false, name);
  if (rc) return rc;
  CCQ_REQUIRE(aligned(x, 16), "%s: x must be 16-byte aligned", name);
  const MoeLayout L = moe_layout(T, k, ex, 2);
  CCQ_REQUIRE(workspace && workspace_bytes >= L.total && aligned(workspace, 256),
              "%s: workspace of %zu bytes (256-byte aligned) needed, %zu given", name, L.total, workspace_bytes);
  return 0;
}

// The routed gate/up launch of a decode batch: routing in every workgroup,
// the schedule, ids and weights written by workgroup 0, the SiLU(gate)*up
// intermediate into the workspace.
static int launch_route_gate_up(const void* x, int x_dtype, const float* logits, int64_t T, int64_t k, int mode,
                                int64_t* ids, float* wts, const ccq_w4_experts* ex, char* ws, const MoeLayout& L,
                                hipStream_t st, int shared = 0, float shared_w = 0.f) {
  const int64_t H = ex->hidden, I = ex->inter, G = ex->group_size;
  W4SP w = {};
  w.x = x;
  w.ldx = H;
  w.row_div = (int)(k + shared);
  w.w0 = (const uint32_t*)ex->w_gate;
  w.sz0 = ex->sz_gate;
  w.w1 = (const uint32_t*)ex->w_up;
  w.sz1 = ex->sz_up;
  w.szw = (int)sz_words_per_column(H, G);
  w.w_es = H * I / 8;
  w.sz_es = I * w.szw;
  w.y = ws + L.off_inter;
  w.ldy = I;
  w.y_dtype = x_dtype;
  w.N = (int)I;
  w.K = (int)H;
  w.KT = (int)(H / 128);
  w.nib_mask = 0x000F000Fu;
  w.logits = logits;
  w.rT = (int)T;
  w.rE = (int)(ex->num_experts - shared);
  w.rk = (int)k;
  w.rmode = mode;
  w.rshared = shared;
  w.rshared_w = shared_w;
  w.ids_out = ids;
  w.wts_out = wts;
  w.sched_rows = (int32_t*)(ws + L.off_sorted);
  w.sched_tile_expert = (int32_t*)(ws + L.off_tile_expert);
  w.sched_meta = (int32_t*)(ws + L.off_meta);
  w.sched_counts = (int32_t*)(ws + L.off_counts);
  return launch_stream<EPI_SILU>(w, 2, x_dtype == CCQ_BF16, ex->scale_dtype == CCQ_BF16, L.max_tiles, st);
}

// The down stage and the combine of a decode batch of at most RD_MAXA
// assignments in one launch, on the schedule the routed gate/up stage
// published: one workgroup per 16 output columns takes that block of every
// routed expert (the assignments' intermediate rows are its MFMA rows) and
// writes y as moe_combine_kernel does, bit for bit (each row's products are
// the down stage's, and the slots are summed in the same order).
static bool route_down_fits(const ccq_w4_experts* ex, int64_t T, int64_t ks) {
  return T * ks <= RD_MAXA && ex->group_size == 128 && ex->hidden % 16 == 0 && ex->inter % 128 == 0 &&
         ex->inter / 128 <= 16;
}

static int launch_route_down(const void* inter, int x_dtype, int64_t T, int64_t ks, const int64_t* ids,
                             const float* wts, void* y, int y_dtype, const ccq_w4_experts* ex, char* ws,
                             const MoeLayout& L, hipStream_t st) {
  const int64_t H = ex->hidden, I = ex->inter, G = ex->group_size;
  W4SP w = {};
  w.x = inter;
  w.ldx = I;
  w.rows = (const int32_t*)(ws + L.off_sorted);
  w.row_div = 1;
  w.tile_expert = (const int32_t*)(ws + L.off_tile_expert);
  w.meta = (const int32_t*)(ws + L.off_meta);
  w.tiles = (int)L.max_tiles;
  w.w0 = (const uint32_t*)ex->w_down;
  w.sz0 = ex->sz_down;
  w.szw = (int)sz_words_per_column(I, G);
  w.w_es = I * H / 8;
  w.sz_es = H * w.szw;
  w.N = (int)H;
  w.K = (int)I;
  w.KT = (int)(I / 128);
  w.nib_mask = 0x000F000Fu;
  w.rT = (int)(T * ks);
  w.cwts = wts;
  w.cids = ids;
  w.cE = ex->num_experts;
  w.cy = y;
  w.ldcy = H;
  w.cy_dtype = y_dtype;
  w.cT = (int)T;
  w.ck = (int)ks;
  const dim3 grid((unsigned)(H / 16)), block(512);
  const bool xb = x_dtype == CCQ_BF16, sb = ex->scale_dtype == CCQ_BF16;
  if (xb) {
    if (sb)
      launch((w4_stream_kernel<__bf16, __bf16, EPI_ROWS, 2, 1, true>), grid, block, 0, st, w);
    else
      launch((w4_stream_kernel<__bf16, _Float16, EPI_ROWS, 2, 1, true>), grid, block, 0, st, w);
  } else {
    if (sb)
      launch((w4_stream_kernel<_Float16, __bf16, EPI_ROWS, 2, 1, true>), grid, block, 0, st, w);
    else
      launch((w4_stream_kernel<_Float16, _Float16, EPI_ROWS, 2, 1, true>), grid, block, 0, st, w);
  }
  return launch_status("w4 routed down + combine");
}

extern "C" int ccq_moe_w4_route_gate_up(const void* x, int x_dtype, const float* logits, int64_t T, int64_t k,
                                        int mode, int64_t* ids_out, float* weights_out, const ccq_w4_experts* ex,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_forward_args("ccq_moe_w4_route_gate_up", x, x_dtype, logits, T, k, mode, nullptr, CCQ_F32, ex,
                              workspace, workspace_bytes, false);
  if (rc || T == 0) return rc;
  const MoeLayout L = moe_layout(T, k, ex, 2);
  if (!fused_route(L, ex, k)) {
    set_error("ccq_moe_w4_route_gate_up: T=%lld, k=%lld is not a decode batch routed in the gate/up kernel",
              (long long)T, (long long)k);
    return CCQ_EUNSUPPORTED;
  }
  char* ws = (char*)workspace;
  int64_t* ids = ids_out != nullptr ? ids_out : (int64_t*)(ws + L.off_ids);
  float* wts = weights_out != nullptr ? weights_out : (float*)(ws + L.off_wts);
  return launch_route_gate_up(x, x_dtype, logits, T, k, mode, ids, wts, ex, ws, L, as_stream(stream));
}

extern "C" int ccq_moe_w4_forward(const void* x, int x_dtype, const float* logits, int64_t T, int64_t k, int mode,
                                  int64_t* ids_out, float* weights_out, void* y, int y_dtype,
                                  const ccq_w4_experts* ex, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_forward_args("ccq_moe_w4_forward", x, x_dtype, logits, T, k, mode, y, y_dtype, ex, workspace,
                              workspace_bytes, true);
  if (rc || T == 0) return rc;
  const MoeLayout L = moe_layout(T, k, ex, 2);
  hipStream_t st = as_stream(stream);
  char* ws = (char*)workspace;
  int64_t* ids = ids_out != nullptr ? ids_out : (int64_t*)(ws + L.off_ids);
  float* wts = weights_out != nullptr ? weights_out : (float*)(ws + L.off_wts);
  if (!fused_route(L, ex, k)) {  // separate routing kernel, then the FFN
    rc = ccq_topk_softmax(logits, wts, ids, T, ex->num_experts, k, mode, stream);
    if (rc) return rc;
    return ccq_moe_w4_ffn(x, x_dtype, ids, wts, y, y_dtype, T, k, ex, workspace, workspace_bytes, stream);
  }
  const int64_t H = ex->hidden;
  int32_t* sorted = (int32_t*)(ws + L.off_sorted);
  int32_t* tile_expert = (int32_t*)(ws + L.off_tile_expert);
  int32_t* meta = (int32_t*)(ws + L.off_meta);
  void* inter = ws + L.off_inter;
  float* rows = (float*)(ws + L.off_rows);
  // gate/up + SiLU with the routing done inside its workgroups
  rc = launch_route_gate_up(x, x_dtype, logits, T, k, mode, ids, wts, ex, ws, L, st);
  if (rc) return rc;
  if (route_down_fits(ex, T, k))  // down and combine in one launch
    return launch_route_down(inter, x_dtype, T, k, ids, wts, y, y_dtype, ex, ws, L, st);
  rc = run_down(inter, x_dtype, sorted, tile_expert, meta, L.max_tiles, rows, ex, st);
  if (rc) return rc;
  return launch_combine(rows, CCQ_F32, wts, ids, ex->num_experts, y, y_dtype, T, k, H, st);
}

// ids / weights [T, k] -> [T, k + 1], the shared expert's slot (expert E,
// weight g) last
__global__ void append_shared_slot_kernel(const int64_t* __restrict__ ids, const float* __restrict__ wts,
                                          int64_t* __restrict__ ids2, float* __restrict__ wts2, int64_t T, int64_t k,
                                          int64_t E, float g) {
  const int64_t ks = k + 1;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < T * ks; i += stride) {
    const int64_t t = i / ks, j = i - t * ks;
    ids2[i] = j < k ? ids[t * k + j] : E;
    wts2[i] = j < k ? wts[t * k + j] : g;
  }
}

extern "C" int ccq_moe_w4_forward_shared(const void* x, int x_dtype, const float* logits, int64_t T, int64_t k,
                                         int mode, float shared_gate, int64_t* ids_out, float* weights_out, void* y,
                                         int y_dtype, const ccq_w4_experts* ex, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  const char* name = "ccq_moe_w4_forward_shared";
  int rc = check_experts(ex, name);
  if (rc) return rc;
  CCQ_REQUIRE(ex->num_experts >= 2, "%s: the stack holds the routed experts and the shared expert last", name);
  CCQ_REQUIRE(k >= 1 && k <= 15 && k < ex->num_experts, "%s: bad k=%lld for %lld routed experts", name,
              (long long)k, (long long)(ex->num_experts - 1));
  const int64_t ks = k + 1, Er = ex->num_experts - 1;
  CCQ_REQUIRE(T >= 0 && T * ks <= 65536 && T <= 65535, "%s: bad T=%lld", name, (long long)T);
  // the checks of ccq_moe_w4_forward with k + 1 slots (workspace included)
  rc = check_forward_args(name, x, x_dtype, logits, T, ks, mode, y, y_dtype, ex, workspace, workspace_bytes, true);
  if (rc || T == 0) return rc;
  const MoeLayout L = moe_layout(T, ks, ex, 2);
  hipStream_t st = as_stream(stream);
  char* ws = (char*)workspace;
  int64_t* ids = ids_out != nullptr ? ids_out : (int64_t*)(ws + L.off_ids);
  float* wts = weights_out != nullptr ? weights_out : (float*)(ws + L.off_wts);
  if (!fused_route(L, ex, ks)) {
    // routing over the Er logits into the (not yet used) down-row area,
    // then the shared slot appended, then the FFN with k + 1 slots
    int64_t* tids = (int64_t*)(ws + L.off_rows);
    float* twts = (float*)(ws + L.off_rows + align256((size_t)(T * k) * 8));
    rc = ccq_topk_softmax(logits, twts, tids, T, Er, k, mode, stream);
    if (rc) return rc;
    launch(append_shared_slot_kernel, dim3(grid_for(T * ks, 256)), dim3(256), 0, st, tids, twts, ids,
                       wts, T, k, Er, shared_gate);
    rc = launch_status(name);
    if (rc) return rc;
    return ccq_moe_w4_ffn(x, x_dtype, ids, wts, y, y_dtype, T, ks, ex, workspace, workspace_bytes, stream);
  }
  int32_t* sorted = (int32_t*)(ws + L.off_sorted);
  int32_t* tile_expert = (int32_t*)(ws + L.off_tile_expert);
  int32_t* meta = (int32_t*)(ws + L.off_meta);
  void* inter = ws + L.off_inter;
  float* rows = (float*)(ws + L.off_rows);
  rc = launch_route_gate_up(x, x_dtype, logits, T, k, mode, ids, wts, ex, ws, L, st, 1, shared_gate);
  if (rc) return rc;
  if (route_down_fits(ex, T, ks))  // down and combine in one launch
    return launch_route_down(inter, x_dtype, T, ks, ids, wts, y, y_dtype, ex, ws, L, st);
  rc = run_down(inter, x_dtype, sorted, tile_expert, meta, L.max_tiles, rows, ex, st);
  if (rc) return rc;
  return launch_combine(rows, CCQ_F32, wts, ids, ex->num_experts, y, y_dtype, T, ks, ex->hidden, st);
}

// ---------------------------------------------------------------------------
// ccq_moe_w4_forward without a caller workspace.  The schedule, intermediate
// and down rows go to `scratch`, a file-scope device array: every GPU the
// library runs on holds its own copy (CCQ_MOE_W4_NOALLOC_BYTES) until the
// process ends.  Its device address is looked up once per device with that
// device current; the array's name is only a host-side stand-in and is never
// passed to a kernel.  Nothing here allocates, and nothing in the workspace
// needs initial contents (every kernel writes what it later reads), so no
// clear is issued.  Calls that overlap in time on one GPU share the array
// and race.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[CCQ_MOE_W4_NOALLOC_BYTES];

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};

// Device address of `scratch` on the current device.
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("ccq_moe_w4_forward_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  CCQ_REQUIRE(dev >= 0 && dev < kScratchDevices, "ccq_moe_w4_forward_noalloc: device %d outside [0, %d)", dev,
              kScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("ccq_moe_w4_forward_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
      return e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace

extern "C" int ccq_moe_w4_forward_noalloc(const void* x, int x_dtype, const float* logits, int64_t T, int64_t k,
                                          int mode, int64_t* ids_out, float* weights_out, void* y, int y_dtype,
                                          const ccq_w4_experts* ex, void* stream) {
  int rc = check_experts(ex, "ccq_moe_w4_forward_noalloc");
  if (rc) return rc;
  CCQ_REQUIRE(T >= 0 && k >= 1 && k <= 16 && k <= ex->num_experts,
              "ccq_moe_w4_forward_noalloc: bad T=%lld / k=%lld", (long long)T, (long long)k);
  CCQ_REQUIRE(T * k <= 65536 && T <= 65535, "ccq_moe_w4_forward_noalloc: T=%lld too large", (long long)T);
  if (T == 0) return 0;
  const size_t need = moe_layout(T, k, ex, 2).total;
  CCQ_REQUIRE(need <= (size_t)CCQ_MOE_W4_NOALLOC_BYTES,
              "ccq_moe_w4_forward_noalloc: T=%lld, k=%lld on this layer needs %zu bytes of scratch, the maximum "
              "is %zu", (long long)T, (long long)k, need, (size_t)CCQ_MOE_W4_NOALLOC_BYTES);
  void* ws = nullptr;
  rc = scratch_address(&ws);
  if (rc) return rc;
  return ccq_moe_w4_forward(x, x_dtype, logits, T, k, mode, ids_out, weights_out, y, y_dtype, ex, ws,
                            (size_t)CCQ_MOE_W4_NOALLOC_BYTES, stream);
}
