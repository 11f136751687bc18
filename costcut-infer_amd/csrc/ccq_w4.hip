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

#include <math.h>

namespace ccq {

int launch_align(const int64_t* ids, int64_t n, int64_t E, int64_t tile_m, int32_t* sorted_ids,
                 int32_t* tile_expert, int32_t* meta, int32_t* counts, hipStream_t st);
int launch_combine(const float* rows, const float* wts, const int64_t* ids, int64_t E, void* y, int y_dtype,
                   int64_t T, int64_t k, int64_t H, hipStream_t st);

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

template <typename AT>
__device__ __forceinline__ typename Act<AT>::vec dq_b(uint32_t w) {
  u32x4 r;
  r[0] = (w & 0x000F000Fu) | Act<AT>::kMagic2;
  r[1] = ((w >> 4) & 0x000F000Fu) | Act<AT>::kMagic2;
  r[2] = ((w >> 8) & 0x000F000Fu) | Act<AT>::kMagic2;
  r[3] = ((w >> 12) & 0x000F000Fu) | Act<AT>::kMagic2;
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
    hipLaunchKernelGGL((w4_skinny_kernel<AT, ST, NB, 4, EPI>), grid, block, lds, st, p);
  else if (G == 64)
    hipLaunchKernelGGL((w4_skinny_kernel<AT, ST, NB, 2, EPI>), grid, block, lds, st, p);
  else if constexpr (NB <= 2)  // plan_skinny never pairs 4 column tiles with G = 32
    hipLaunchKernelGGL((w4_skinny_kernel<AT, ST, NB, 1, EPI>), grid, block, lds, st, p);
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

// ------------------------------------------------ prefill grouped GEMM --
// For tiles with many rows (prefill, experts receiving tens to thousands of
// tokens): a workgroup of 8 waves computes a BM-row tile x 128 output
// columns, wave w owning the 16 columns of weight tile nb*8 + w (gate and up
// for EPI_SILU).  Group size 128 = one k-tile, so per k-tile
//     acc += s * (sum_k x * (MAGIC + q) - (MAGIC + z) * sum_k x)
// with sum_k x of each row formed while the activation tile is staged.
// The activation tile (BM x 128, bf16/fp16) goes through LDS, double-buffered
// one k-tile ahead; the wave's packed weights go straight to registers one
// k-tile ahead and are dequantized there (one AND/OR per weight pair).
struct W4GP {
  const void* x;
  int64_t ldx;
  const int32_t* rows;         // per tile BM row ids (-1 = padding); null = dense rows
  int row_div;                 // activation row = row id / row_div
  const int32_t* tile_expert;  // null = one weight
  const int32_t* meta;         // meta[0] = valid schedule tiles; null = all
  int tile_div;                // kernel tiles per schedule tile (schedule rows / BM)
  const uint32_t* w0;
  const uint32_t* sz0;
  const uint32_t* w1;          // up projection (EPI_SILU)
  const uint32_t* sz1;
  int64_t w_es, sz_es;         // per-expert strides (words)
  void* y;
  int64_t ldy;
  int y_dtype;
  int M, N, K, KT, szw;
};

constexpr int WG_BM_SMALL = 64;
constexpr int WG_BM_LARGE = 128;
constexpr int WG_WAVES = 8;
constexpr int WG_ALD = 128 + 8;  // LDS row stride of the activation tile (elements)

template <typename AT, typename ST, int EPI, int BM>
__global__ __launch_bounds__(512) void w4_group_gemm_kernel(const W4GP p) {
  using V = typename Act<AT>::vec;
  constexpr int NQ = EPI == EPI_SILU ? 2 : 1;
  constexpr int RT = BM / 16;
  constexpr int AP = BM * 16 / (64 * WG_WAVES);  // 16-byte activation pieces per thread
  __shared__ __align__(16) AT As[2][BM * WG_ALD];
  __shared__ __align__(16) float Sx[2][BM];
  __shared__ int Rid[BM];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nb = blockIdx.x, tile = blockIdx.y;
  if (p.meta != nullptr && tile >= p.meta[0] * p.tile_div) return;
  const int ex = p.tile_expert ? p.tile_expert[tile / p.tile_div] : 0;
  if (tid < BM) {
    int rid;
    if (p.rows) {
      rid = p.rows[tile * BM + tid];
    } else {
      rid = tile * BM + tid;
      if (rid >= p.M) rid = -1;
    }
    Rid[tid] = rid;
  }
  if (!__syncthreads_or(tid < BM && Rid[tid] >= 0)) return;

  // activation staging: piece i = tid + 512*j covers row i / 16, elements
  // 8*(i % 16) .. +8 of the k-tile; the 16 pieces of a row sit in 16
  // consecutive lanes, which also reduce the row sum
  const AT* asrc[AP];
  bool aval[AP];
#pragma unroll
  for (int j = 0; j < AP; ++j) {
    const int i = tid + 64 * WG_WAVES * j, row = i >> 4, part = i & 15;
    aval[j] = Rid[row] >= 0;
    asrc[j] = reinterpret_cast<const AT*>(p.x) + (int64_t)(aval[j] ? Rid[row] / p.row_div : 0) * p.ldx + 8 * part;
  }
  struct AStage {
    u32x4 v[AP];
  };
  auto load_a = [&](AStage& st, int kt) {
#pragma unroll
    for (int j = 0; j < AP; ++j) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(asrc[j] + (int64_t)kt * 128);
      st.v[j] = aval[j] ? v : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_a = [&](const AStage& st, int buf) {
#pragma unroll
    for (int j = 0; j < AP; ++j) {
      const int i = tid + 64 * WG_WAVES * j, row = i >> 4, part = i & 15;
      *reinterpret_cast<u32x4*>(&As[buf][row * WG_ALD + 8 * part]) = st.v[j];
      const V a = __builtin_bit_cast(V, st.v[j]);
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) sum += (float)a[e];
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) sum += __shfl_xor(sum, off, 64);
      if (part == 0) Sx[buf][row] = sum;
    }
  };

  // the wave's weight column tile (16 columns) of each matrix
  const int nt = nb * WG_WAVES + wave;
  const int r = lane & 15, kq = lane >> 4;
  const uint32_t* wsrc[NQ];
  const uint32_t* zsrc[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    wsrc[q] = (q == 0 ? p.w0 : p.w1) + (int64_t)ex * p.w_es + (int64_t)nt * p.KT * 256 + lane * 4;
    zsrc[q] = (q == 0 ? p.sz0 : p.sz1) + (int64_t)ex * p.sz_es + (int64_t)(nt * 16 + r) * p.szw;
  }
  struct BStage {
    u32x4 w[NQ];
    uint32_t z[NQ];
  };
  auto load_b = [&](BStage& st, int kt) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      st.w[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wsrc[q] + (int64_t)kt * 256));
      st.z[q] = zsrc[q][kt];
    }
  };

  f32x4 acc[RT][NQ];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int q = 0; q < NQ; ++q) acc[rt][q] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int buf, const BStage& b) {
    V bw[NQ][4];
    float s[NQ], c[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
#pragma unroll
      for (int j = 0; j < 4; ++j) bw[q][j] = dq_b<AT>(b.w[q][j]);
      s[q] = sz_scale<ST>(b.z[q]);
      c[q] = Act<AT>::kMagic + (float)(b.z[q] >> 16);
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      V a[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) a[j] = *reinterpret_cast<const V*>(&As[buf][(rt * 16 + r) * WG_ALD + 32 * j + 8 * kq]);
      const f32x4 sx = *reinterpret_cast<const f32x4*>(&Sx[buf][rt * 16 + 4 * kq]);
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) t = mfma16(a[j], bw[q][j], t);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[rt][q][i] = fmaf(s[q], fmaf(-c[q], sx[i], t[i]), acc[rt][q][i]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // pipeline: k-tile kt computes from LDS buffer kt & 1 and weight stage
  // kt & 1 while the activations of kt+1 (issued first) and the weights of
  // kt+1 are in flight
  AStage as0, as1;
  BStage bs0, bs1;
  load_a(as0, 0);
  load_b(bs0, 0);
  store_a(as0, 0);
  __syncthreads();
  for (int kt = 0; kt < p.KT; kt += 2) {
    if (kt + 1 < p.KT) {
      load_a(as1, kt + 1);
      load_b(bs1, kt + 1);
    }
    compute(0, bs0);
    if (kt + 1 < p.KT) store_a(as1, 1);
    __syncthreads();
    if (kt + 1 >= p.KT) break;
    if (kt + 2 < p.KT) {
      load_a(as0, kt + 2);
      load_b(bs0, kt + 2);
    }
    compute(1, bs1);
    if (kt + 2 < p.KT) store_a(as0, 0);
    __syncthreads();
  }

  // epilogue: lane holds rows rt*16 + 4*kq + i of column nt*16 + r
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rid = Rid[rt * 16 + 4 * kq + i];
      if (rid < 0) continue;
      const int64_t o = (int64_t)rid * p.ldy + nt * 16 + r;
      if (EPI == EPI_SILU) {
        const float g = acc[rt][0][i], u = acc[rt][NQ - 1][i];
        store_val(p.y, o, g / (1.0f + expf(-g)) * u, p.y_dtype);
      } else {
        store_val(p.y, o, acc[rt][0][i], p.y_dtype);
      }
    }
}

// bm: rows per schedule tile.  Gate/up (two matrices) runs 64-row kernel
// tiles (128 would spill registers), splitting 128-row schedule tiles.
template <int EPI>
static int launch_group_gemm(W4GP p, int x_bf16, int s_bf16, int bm, int64_t tiles, hipStream_t st) {
  const int kbm = EPI == EPI_SILU ? WG_BM_SMALL : bm;
  p.tile_div = bm / kbm;
  bm = kbm;
  const dim3 grid((unsigned)(p.N / 128), (unsigned)(tiles * p.tile_div)), block(64 * WG_WAVES);
#define CCQ_LAUNCH_GG(AT, ST)                                                                     \
  do {                                                                                            \
    if constexpr (EPI != EPI_SILU) {                                                              \
      if (bm == WG_BM_LARGE) {                                                                    \
        hipLaunchKernelGGL((w4_group_gemm_kernel<AT, ST, EPI, WG_BM_LARGE>), grid, block, 0, st, p); \
        break;                                                                                    \
      }                                                                                           \
    }                                                                                             \
    hipLaunchKernelGGL((w4_group_gemm_kernel<AT, ST, EPI, WG_BM_SMALL>), grid, block, 0, st, p);  \
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

// Tile rows of the grouped kernel for n assignments over E experts (each
// tile streams its expert's weights, so a tile should hold all of them).
static int group_tile_rows(int64_t n, int64_t E) { return n >= 32 * E ? WG_BM_LARGE : WG_BM_SMALL; }
// The grouped kernel replaces the 16-row decode kernel once the average
// expert receives at least 16 rows (and the shape suits it: group 128,
// N a multiple of 128).
static bool use_group_gemm(int64_t n, int64_t E, int64_t G, int64_t N1, int64_t N2) {
  return n >= 16 * E && G == 128 && N1 % 128 == 0 && N2 % 128 == 0;
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
  hipLaunchKernelGGL(awq_dequant_kernel, dim3(grid1d(K * N / 8)), dim3(256), 0, as_stream(stream),
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
  hipLaunchKernelGGL(awq_repack_kernel, dim3(grid1d(K * N / 8)), dim3(256), 0, as_stream(stream),
                     (const uint32_t*)qweight, (uint32_t*)tiled, K, N);
  return launch_status("ccq_awq_repack");
}

extern "C" int ccq_awq_unpack_tiled(const int32_t* tiled, int32_t* qweight, int64_t K, int64_t N, void* stream) {
  CCQ_REQUIRE(K >= 0 && N >= 0, "ccq_awq_unpack_tiled: negative shape");
  CCQ_REQUIRE(K % 128 == 0 && N % 16 == 0, "ccq_awq_unpack_tiled: need K %% 128 == 0 and N %% 16 == 0");
  if (K == 0 || N == 0) return 0;
  CCQ_REQUIRE(qweight && tiled, "ccq_awq_unpack_tiled: null pointer");
  CCQ_REQUIRE((const void*)qweight != (const void*)tiled, "ccq_awq_unpack_tiled: in-place is not supported");
  hipLaunchKernelGGL(awq_unpack_tiled_kernel, dim3(grid1d(K * N / 8)), dim3(256), 0, as_stream(stream),
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
  hipLaunchKernelGGL(awq_pack_sz_kernel, dim3(grid1d(N * sz_words_per_column(K, group_size))), dim3(256), 0,
                     as_stream(stream), (const uint32_t*)qzeros, (const uint16_t*)scales, sz, K, N, group_size);
  return launch_status("ccq_awq_pack_sz");
}

extern "C" int ccq_w4_gemm(const void* x, int x_dtype, const int32_t* w_tiled, const uint32_t* sz, int scale_dtype,
                           void* y, int y_dtype, int64_t M, int64_t K, int64_t N, int64_t group_size,
                           void* stream) {
  CCQ_REQUIRE(M >= 0 && K >= 0 && N >= 0, "ccq_w4_gemm: negative shape");
  CCQ_REQUIRE(K % 128 == 0 && N % 16 == 0, "ccq_w4_gemm: need K %% 128 == 0 and N %% 16 == 0 (K=%lld N=%lld)",
              (long long)K, (long long)N);
  CCQ_REQUIRE(valid_group(group_size), "ccq_w4_gemm: group_size=%lld not in {32, 64, 128}", (long long)group_size);
  CCQ_REQUIRE(x_dtype == CCQ_F16 || x_dtype == CCQ_BF16, "ccq_w4_gemm: x_dtype must be f16|bf16");
  CCQ_REQUIRE(scale_dtype == CCQ_F16 || scale_dtype == CCQ_BF16, "ccq_w4_gemm: scale_dtype must be f16|bf16");
  CCQ_REQUIRE(y_dtype == CCQ_F16 || y_dtype == CCQ_BF16 || y_dtype == CCQ_F32, "ccq_w4_gemm: bad y_dtype");
  CCQ_REQUIRE(M > 64 || cdiv(M, 16) <= 65535, "ccq_w4_gemm: M=%lld too large", (long long)M);
  CCQ_REQUIRE(K <= (1 << 20) && N / 16 <= 0x7fffffff, "ccq_w4_gemm: K=%lld or N=%lld too large", (long long)K,
              (long long)N);
  if (M == 0 || N == 0) return 0;
  CCQ_REQUIRE(K > 0, "ccq_w4_gemm: K == 0");
  CCQ_REQUIRE(x && w_tiled && sz && y, "ccq_w4_gemm: null pointer");
  CCQ_REQUIRE(aligned(x, 16) && aligned(w_tiled, 16) && aligned(sz, 16),
              "ccq_w4_gemm: x, w_tiled and sz must be 16-byte aligned");
  if (M > 64 && group_size == 128 && N % 128 == 0) {
    // prefill-sized: tiles of 64/128 rows stream the weight once per tile
    const int bm = M >= WG_BM_LARGE ? WG_BM_LARGE : WG_BM_SMALL;
    CCQ_REQUIRE(cdiv(M, bm) <= 65535, "ccq_w4_gemm: M=%lld too large", (long long)M);
    W4GP g = {};
    g.x = x;
    g.ldx = K;
    g.row_div = 1;
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
    CCQ_REQUIRE(cdiv(M, bm) <= 65535, "ccq_w4_gemm: M=%lld too large", (long long)M);
    return launch_group_gemm<EPI_STORE>(g, x_dtype == CCQ_BF16, scale_dtype == CCQ_BF16, bm, cdiv(M, bm),
                                        as_stream(stream));
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
  int tile_m;       // rows per schedule tile: 16 (decode kernel) or 64/128 (grouped kernel)
  bool grouped;
  size_t off_sorted, off_tile_expert, off_meta, off_counts, off_inter, off_rows, total;
};

MoeLayout moe_layout(int64_t T, int64_t k, const ccq_w4_experts* ex, int x_bytes) {
  MoeLayout L;
  L.n = T * k;
  L.grouped = use_group_gemm(L.n, ex->num_experts, ex->group_size, ex->inter, ex->hidden);
  L.tile_m = L.grouped ? group_tile_rows(L.n, ex->num_experts) : 16;
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
  L.total = o;
  return L;
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

extern "C" int ccq_moe_w4_ffn(const void* x, int x_dtype, const int64_t* ids, const float* weights, void* y,
                              int y_dtype, int64_t T, int64_t k, const ccq_w4_experts* ex, void* workspace,
                              size_t workspace_bytes, void* stream) {
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
  rc = launch_align(ids, L.n, ex->num_experts, L.tile_m, sorted, tile_expert, meta, counts, st);
  if (rc) return rc;
  if (L.grouped) {
    const int64_t H = ex->hidden, I = ex->inter, G = ex->group_size;
    W4GP g = {};
    g.x = x;
    g.ldx = H;
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
    g.N = (int)I;
    g.K = (int)H;
    g.KT = (int)(H / 128);
    rc = launch_group_gemm<EPI_SILU>(g, x_dtype == CCQ_BF16, ex->scale_dtype == CCQ_BF16, L.tile_m, L.max_tiles, st);
    if (rc) return rc;
    W4GP d = {};
    d.x = inter;
    d.ldx = I;
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
    d.y_dtype = CCQ_F32;
    d.N = (int)H;
    d.K = (int)I;
    d.KT = (int)(I / 128);
    rc = launch_group_gemm<EPI_ROWS>(d, x_dtype == CCQ_BF16, ex->scale_dtype == CCQ_BF16, L.tile_m, L.max_tiles, st);
    if (rc) return rc;
  } else {
    rc = run_gate_up(x, x_dtype, k, sorted, tile_expert, meta, L.max_tiles, inter, ex, st);
    if (rc) return rc;
    rc = run_down(inter, x_dtype, sorted, tile_expert, meta, L.max_tiles, rows, ex, st);
    if (rc) return rc;
  }
  return launch_combine(rows, weights, ids, ex->num_experts, y, y_dtype, T, k, ex->hidden, st);
}
