// FP8 e4m3fn with 128x128 block weight scales and per-token-per-128 dynamic
// activation scales on gfx950: activation quantization, weight re-pack, the
// block-scaled grouped GEMM on v_mfma_f32_32x32x64_f8f6f4, and the MoE
// expert FFN built on it.
//
// Format (public DeepSeek-V3-style block FP8): weights w [N, K] e4m3fn bytes
// (row = output channel) with s_w [N/128, K/128] float32,
// W[n, k] = fp8(w[n, k]) * s_w[n/128, k/128]; activations x [T, K] quantized
// per token per 128 channels: s_a = max(amax, 1e-12) / 448 (float32),
// q = RNE(x / s_a) saturated to +-448.  Two 32x32x64 MFMAs cover one
// 128-wide K block, so each block's product is scaled once on the
// accumulator: acc += (s_a[row, kb] * s_w[nb, kb]) * mfma(q_a, q_w).
//
// Weight tile layout: tile (nt, kb) = 16 output channels x 128 K bytes =
// 2 KiB at byte (nt*KB + kb)*2048; inside, [half h][lane l][16 bytes] with
// bytes k = kb*128 + 32*(l >> 4) + 16*h + e of channel nt*16 + (l & 15).
// Each half is one contiguous 1 KiB copy.  The 32x32x64 B operand of lane
// (h', c) = (l >> 5, l & 31) at K step s (bytes 64s + 32h' .. +32) is the
// two halves of the slot of lane 16*(2s + h') + (c & 15) in 16-column tile
// c >> 4; the A operand (row c, same K bytes) reads the activation tile.
#include "ccq_common.h"

#include <math.h>

#include <type_traits>

namespace ccq {

constexpr float kFp8Max = 448.0f;
constexpr float kAmaxFloor = 1e-12f;

__device__ __forceinline__ float load_as_f32(const void* x, int64_t i, int dt) {
  if (dt == CCQ_F32) return reinterpret_cast<const float*>(x)[i];
  const uint32_t b = reinterpret_cast<const uint16_t*>(x)[i];
  return dt == CCQ_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// ---------------------------------------------------- activation quant --
// 16 lanes per (row, 128-column block), 8 columns per lane.
template <int XT>
__global__ __launch_bounds__(256) void fp8_act_quant_kernel(const void* __restrict__ x, int64_t ldx,
                                                            uint8_t* __restrict__ q, int64_t ldq,
                                                            float* __restrict__ s, int64_t lds_, int64_t rows,
                                                            int64_t KB) {
  const int lane = threadIdx.x & 63;
  const int sub = lane & 15;
  const int64_t nblk = rows * KB;
  const int64_t stride = (int64_t)gridDim.x * 16;
  for (int64_t b = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4; b < nblk; b += stride) {
    const int64_t row = (int64_t)((uint32_t)b / (uint32_t)KB), kb = b - row * KB;  // rows * KB < 2^31
    const int64_t c0 = kb * 128 + 8 * sub;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = load_as_f32(x, row * ldx + c0 + e, XT);
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const float sc = fmaxf(amax, kAmaxFloor) / kFp8Max;
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) lo |= f32_to_fp8_rne(v[e] / sc) << (8 * e);
#pragma unroll
    for (int e = 0; e < 4; ++e) hi |= f32_to_fp8_rne(v[4 + e] / sc) << (8 * e);
    *reinterpret_cast<uint2*>(q + row * ldq + c0) = make_uint2(lo, hi);
    if (sub == 0) s[row * lds_ + kb] = sc;
  }
}

// The same with 16-byte loads (x 16-byte aligned, ldx a multiple of 8 bf16 /
// f16 or 4 float32 values), the 16-lane amax on DPP moves (max is a
// selection, so the order of the steps does not change it) and the
// hardware RNE conversion (v_cvt_pk_fp8_f32, equal to f32_to_fp8_rne for
// every |v| <= 460; here |v| <= 448 (1 + 2^-22)); a lane with a NaN among
// its quotients (a NaN or infinite input) encodes them in software (NaN ->
// 0x7F whatever its sign).
template <int XT>
__global__ __launch_bounds__(256) void fp8_act_quant_vec_kernel(const void* __restrict__ x, int64_t ldx,
                                                                uint8_t* __restrict__ q, int64_t ldq,
                                                                float* __restrict__ s, int64_t lds_,
                                                                int64_t rows, int64_t KB) {
  const int lane = threadIdx.x & 63;
  const int sub = lane & 15;
  const int64_t nblk = rows * KB;
  const int64_t stride = (int64_t)gridDim.x * 16;
  for (int64_t b = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4; b < nblk; b += stride) {
    const int64_t row = (int64_t)((uint32_t)b / (uint32_t)KB), kb = b - row * KB;  // rows * KB < 2^31
    const int64_t c0 = kb * 128 + 8 * sub;
    float v[8];
    if constexpr (XT == CCQ_F32) {
      const f32x4* xp = reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(x) + row * ldx + c0);
      const f32x4 a = xp[0], c = xp[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = a[e];
        v[4 + e] = c[e];
      }
    } else {
      const u32x4 w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(x) + row * ldx + c0);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t h = (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
        v[e] = XT == CCQ_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
      }
    }
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
    amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(amax), 0xB1, 0xf, 0xf, false)));
    amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(amax), 0x4E, 0xf, 0xf, false)));
    amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(amax), 0x124, 0xf, 0xf, false)));
    amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(amax), 0x128, 0xf, 0xf, false)));
    const float sc = fmaxf(amax, kAmaxFloor) / kFp8Max;
    float d[8];
    bool nan = false;  // a NaN or infinite input makes a NaN quotient
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      d[e] = v[e] / sc;
      nan = nan || d[e] != d[e];
    }
    uint32_t lo, hi;
    if (!nan) {
      int a = __builtin_amdgcn_cvt_pk_fp8_f32(d[0], d[1], 0, false);
      lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(d[2], d[3], a, true);
      int c = __builtin_amdgcn_cvt_pk_fp8_f32(d[4], d[5], 0, false);
      hi = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(d[6], d[7], c, true);
    } else {
      lo = 0;
      hi = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) lo |= f32_to_fp8_rne(d[e]) << (8 * e);
#pragma unroll
      for (int e = 0; e < 4; ++e) hi |= f32_to_fp8_rne(d[4 + e]) << (8 * e);
    }
    *reinterpret_cast<uint2*>(q + row * ldq + c0) = make_uint2(lo, hi);
    if (sub == 0) s[row * lds_ + kb] = sc;
  }
}

// ----------------------------------------------------------- re-pack --
// Tiled layout: 2 KiB chunks, one per (16-column tile nt, K block kb), in
// the order [nt / 8][kb][nt % 8]: the 8 tiles of a 128-column block are
// contiguous at each K block (16 KiB), so a workgroup streaming a column
// block reads one contiguous range per K block.  Inside a chunk, piece
// 64 h + l (16 bytes) holds row nt*16 + (l & 15), k = kb*128 + 32 (l >> 4)
// + 16 h.  One thread per piece.
__device__ __forceinline__ void fp8_tiled_piece(int64_t i, int64_t KB, int64_t& n, int64_t& k) {
  const int l = (int)(i & 63), h = (int)((i >> 6) & 1);
  const int64_t chunk = i >> 7, t8 = chunk & 7, rest = chunk >> 3, kb = rest % KB, nt = (rest / KB) * 8 + t8;
  n = nt * 16 + (l & 15);
  k = kb * 128 + 32 * (l >> 4) + 16 * h;
}
// byte offset of chunk (nt, kb) in the tiled layout
__host__ __device__ __forceinline__ int64_t fp8_chunk_off(int64_t nt, int64_t kb, int64_t KB) {
  return (((nt >> 3) * KB + kb) * 8 + (nt & 7)) * 2048;
}

__global__ void fp8_repack_kernel(const uint8_t* __restrict__ w, uint8_t* __restrict__ tiled, int64_t N,
                                  int64_t K) {
  const int64_t KB = K / 128, pieces = N * K / 16;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pieces;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t n, k;
    fp8_tiled_piece(i, KB, n, k);
    *reinterpret_cast<u32x4*>(tiled + i * 16) = *reinterpret_cast<const u32x4*>(w + n * K + k);
  }
}

__global__ void fp8_unpack_kernel(const uint8_t* __restrict__ tiled, uint8_t* __restrict__ w, int64_t N,
                                  int64_t K) {
  const int64_t KB = K / 128, pieces = N * K / 16;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pieces;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t n, k;
    fp8_tiled_piece(i, KB, n, k);
    *reinterpret_cast<u32x4*>(w + n * K + k) = *reinterpret_cast<const u32x4*>(tiled + i * 16);
  }
}

// ------------------------------------------------------ block dequant --
// out[n, k] = fp8(w[n, k]) * s_w[n / 128, k / 128] (float32, one rounding),
// any N and K; s_w [ceil(N/128), ceil(K/128)].  Load-time / per-expert use.
__global__ void fp8_block_dequant_kernel(const uint8_t* __restrict__ w, const float* __restrict__ s_w,
                                         float* __restrict__ out, int64_t N, int64_t K) {
  const int64_t n_el = N * K, KB = (K + 127) / 128;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_el; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i / K, k = i - n * K;
    out[i] = fp8_e4m3_to_f32(w[i]) * s_w[(n >> 7) * KB + (k >> 7)];
  }
}

// ------------------------------------------------------ grouped GEMM --
// Persistent grouped GEMM on v_mfma_f32_32x32x64_f8f6f4, the FP8 form of the
// int4 kernel in ccq_w4.hip: one workgroup of 8 waves per compute unit walks
// a list of (128-row tile, column block) items; per 128-wide K block it
// copies from HBM straight into LDS (global_load_lds) the activation tile
// (128 rows x 128 bytes, rows gathered by row id), the weight tiles, the
// rows' activation scales and the block's weight scales, in a ring of three
// K blocks that runs on across items (loads two K blocks ahead).  Waves form
// a 2 (rows) x 4 (columns) grid, each owning 64 rows x 2 tiles of 32
// columns (gate and up for F8_SILU_Q).  Per K block and tile the two MFMAs
// (K = 64 each) give the block's product t and
//     acc += (s_a[row, kb] * s_w[block, kb]) * t.
// Activation rows keep their 16-byte pieces swizzled by row (piece p of row
// r at position p ^ f8_swz(r)), so the operand reads of 16 consecutive rows
// hit 16 different bank groups.
//
// The MoE intermediate h = silu(g) * u is carried between the two stages as
// two e4m3 parts with one scale per row and 128-column block,
//     s = max(amax, 1e-12) / 448,  hi = RNE(h / s),  lo = RNE((h / s - hi) * 16),
// so h = s * (hi + lo / 16) to about 2^-8 relative (a single e4m3 code
// would keep 2^-4, which puts the layer output about 2% away from the float32
// product).  The down stage (F8_ROWS with LO) multiplies both parts by the
// same weight fragments: t = mfma(lo, w) / 16 + mfma(hi, w), one exact
// power-of-two scaling between the two MFMA chains.
enum { F8_STORE = 0, F8_ROWS = 1, F8_SILU_Q = 2 };

struct Fp8GP {
  const uint8_t* a;            // activations e4m3fn [*, K]
  const uint8_t* a_lo;         // LO kernels: their low parts [*, K] (same lda, scaled by 16)
  int64_t lda;
  const float* sa;             // their scales [*, K/128]
  int64_t ldsa;
  const int32_t* rows;         // per tile 128 row ids (-1 = padding, at the end); null = dense rows
  int row_div;                 // activation row = row id / row_div
  const int32_t* tile_expert;  // null = one weight
  const int32_t* meta;         // meta[0] = valid tiles; null = tiles
  int tiles;
  const uint8_t* w0;           // tiled weights (gate for F8_SILU_Q)
  const float* sw0;            // block scales [N/128, K/128]
  const uint8_t* w1;           // up weights for F8_SILU_Q
  const float* sw1;
  int64_t w_es, sw_es;         // per-expert strides (bytes, floats)
  void* y;                     // F8_STORE: [M, N] y_dtype; F8_ROWS: [row id, N] y_dtype
  int64_t ldy;
  int y_dtype;
  uint8_t* qy;                 // F8_SILU_Q: e4m3fn [row id, N] (high and low parts) and scales [row id, N/128]
  uint8_t* qy_lo;
  float* sy;
  int64_t ldqy, ldsy;
  int M, N, K, KB;
};

constexpr int F8_BM = 128;
constexpr int F8_A_BYTES = F8_BM * 128;   // 128 rows x 128 e4m3 bytes
constexpr int F8_STAGES = 3;
constexpr int F8_RID = F8_BM + 64;

// Stage layout: activation tile(s) (the low part after the high one), the
// weight tiles, the rows' activation scales, 2 x 64 copies of block scales.
template <bool LO, int NBT>
struct F8Stage {
  static constexpr int A = F8_A_BYTES * (LO ? 2 : 1);
  static constexpr int B_OFF = A;
  static constexpr int SA_OFF = B_OFF + NBT * 2048;
  static constexpr int SW_OFF = SA_OFF + F8_BM * 4;
  static constexpr int BYTES = SW_OFF + 2 * 256;
};
constexpr size_t f8_lds_bytes(int stage) { return (size_t)F8_STAGES * stage + 3 * F8_RID * 4 + 5 * F8_BM * 4; }
static_assert(f8_lds_bytes(F8Stage<false, 16>::BYTES) <= 160 * 1024, "LDS budget of one workgroup");
static_assert(f8_lds_bytes(F8Stage<true, 8>::BYTES) <= 160 * 1024, "LDS budget of one workgroup");

__device__ __forceinline__ int f8_swz(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }

__device__ __forceinline__ f32x16 mfma_f8_32(const i32x8& a, const i32x8& b, f32x16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
// The same product with B scaled by 2^-4 inside the MFMA: E8M0 block scales
// 127 (1.0) for A and 123 (2^-4) for B.
__device__ __forceinline__ f32x16 mfma_f8_32_b16th(const i32x8& a, const i32x8& b, f32x16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 123);
}

template <int EPI, int CTW, bool LO = false>
__global__ __launch_bounds__(512) void fp8_gemm_kernel(const Fp8GP p) {
  constexpr int NQ = EPI == F8_SILU_Q ? 2 : 1;
  constexpr int WGN = 64 * CTW;      // columns per matrix per item
  constexpr int TPM = WGN / 16;      // 16-column weight tiles per matrix
  constexpr int NBT = NQ * TPM;      // weight tiles per K block
  constexpr int BPW = NBT / 4;       // 1 KiB weight copies per wave (2 per tile)
  constexpr int C32 = CTW * NQ / 2;  // 32-column MFMA tiles per wave
  constexpr int CQ = C32 / NQ;
  constexpr int NSW = WGN == 256 || NQ == 2 ? 2 : 1;  // block scales per K block
  static_assert(NBT % 4 == 0 && NBT <= 16 && C32 >= 1 && C32 <= 2, "tile shape");
  static_assert(!LO || EPI == F8_ROWS, "low activation parts feed the down stage only");
  using SL = F8Stage<LO, NBT>;
  constexpr int F8_STAGE = SL::BYTES, F8_B_OFF = SL::B_OFF, F8_SA_OFF = SL::SA_OFF, F8_SW_OFF = SL::SW_OFF;
  constexpr int NA = LO ? 4 : 2;  // activation copies per wave and K block
  __shared__ __align__(16) char smem[F8_STAGES * F8_STAGE];
  __shared__ __align__(16) int Rid[3][F8_RID];
  __shared__ __align__(16) float part[4 * F8_BM];
  __shared__ __align__(16) float amax_s[F8_BM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int mw = wave >> 2, nw = wave & 3;
  const int nblk = p.N / WGN;
  const int ntiles = p.meta != nullptr ? p.meta[0] : p.tiles;
  // static schedule (as in the int4 kernel): row tiles dealt to XCDs
  // round-robin, all column blocks of a tile on one XCD
  const int xcd = blockIdx.x & 7, wx = blockIdx.x >> 3;
  const int nx = ((int)gridDim.x - xcd + 7) >> 3;
  const int items_x = (ntiles > xcd ? (ntiles - xcd + 7) >> 3 : 0) * nblk;
  if (wx >= items_x) return;
  // rounds of nx items in alternating direction, as in the int4 kernel
  auto item_of = [&](int j) { return j * nx + ((j & 1) ? nx - 1 - wx : wx); };
  const int nmine = items_x / nx + (item_of(items_x / nx) < items_x ? 1 : 0);
  const int KB = p.KB;
  const int total = nmine * KB;

  auto tile_of = [&](int j) { return xcd + 8 * (item_of(j) / nblk); };
  // row ids of item j into Rid[j % 3] (+ expert id copies): DMA from the
  // schedule, or the rows of a dense tile; called two items ahead
  auto fetch_rows = [&](int j) {
    if (j >= nmine) return;
    const int tile = tile_of(j);
    if (p.rows != nullptr) {
      const uint32_t dst = lds_addr(&Rid[j % 3][0]);
      if (wave >= 6) dma4(p.rows + (int64_t)tile * F8_BM, (wave - 6) * 256 + lane * 4, dst + (wave - 6) * 256);
      if (wave == 5 && p.tile_expert != nullptr) dma4(p.tile_expert + tile, 0u, dst + F8_BM * 4);
    } else if (wave >= 6) {
      const int r = (wave - 6) * 64 + lane, rid = tile * F8_BM + r;
      Rid[j % 3][r] = rid < p.M ? rid : -1;
    }
  };
  for (int j = 0; j < 2 && j < nmine; ++j) {
    const int tile = tile_of(j);
    if (tid < F8_BM) {
      const int rid = tile * F8_BM + tid;
      Rid[j][tid] = p.rows != nullptr ? p.rows[(int64_t)tile * F8_BM + tid] : (rid < p.M ? rid : -1);
    }
    if (tid == F8_BM) Rid[j][F8_BM] = p.tile_expert != nullptr ? p.tile_expert[tile] : 0;
  }
  __syncthreads();

  // ---- per-item copy plan of this wave ----
  struct Plan {
    uint32_t aoff[2];
    const uint8_t* bsrc[BPW];
    uint32_t soff;
    const float* swsrc;
    int nvalid, nb;
  };
  const bool has_sa = wave == 4 || wave == 5;
  const bool has_sw = wave >= 6 && wave - 6 < NSW;
  const int ncopy = NA + BPW + (has_sa ? 1 : 0) + (has_sw ? 1 : 0);
  auto make_plan = [&](int j, Plan& P) {
    P.nb = item_of(j) % nblk;
    const int* R = Rid[j % 3];
    const int ex = p.tile_expert != nullptr ? __builtin_amdgcn_readfirstlane(R[F8_BM]) : 0;
    P.nvalid = (int)(__popcll(__ballot(R[lane] >= 0)) + __popcll(__ballot(R[64 + lane] >= 0)));
    const int rid0 = R[0];
    // activations: rows 16*wave + 8*i + (lane >> 3); the lane takes piece
    // (lane & 7) ^ f8_swz(row), which lands at position lane & 7
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = 16 * wave + 8 * i + (lane >> 3);
      const int rid = R[row] >= 0 ? R[row] : rid0;
      const int piece = (lane & 7) ^ f8_swz(row);
      P.aoff[i] = (uint32_t)((int64_t)(rid / p.row_div) * p.lda + piece * 16);
    }
    // weights: copy b of the wave = half (b & 1) of tile b >> 1
#pragma unroll
    for (int b2 = 0; b2 < BPW; ++b2) {
      const int b = wave * BPW + b2, t = b >> 1, q = t / TPM, nt = P.nb * TPM + (t - q * TPM);
      P.bsrc[b2] = (q == 0 ? p.w0 : p.w1) + (int64_t)ex * p.w_es + fp8_chunk_off(nt, 0, KB) + (b & 1) * 1024;
    }
    P.soff = 0;
    if (has_sa) {
      const int row = 64 * (wave - 4) + lane;
      const int rid = R[row] >= 0 ? R[row] : rid0;
      P.soff = (uint32_t)((int64_t)(rid / p.row_div) * p.ldsa * 4);
    }
    P.swsrc = nullptr;
    if (has_sw) {
      // SILU: gate (wave 6) and up (wave 7) of block nb; 256-column items:
      // blocks 2nb and 2nb+1
      const int q = NQ == 2 ? wave - 6 : 0;
      const int blk = NQ == 2 ? P.nb : P.nb * (WGN / 128) + (wave - 6);
      P.swsrc = (q == 0 ? p.sw0 : p.sw1) + (int64_t)ex * p.sw_es + (int64_t)blk * KB;
    }
  };
  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](const Plan& P, int kb, int slot) {
    const uint32_t st = lds0 + slot * F8_STAGE;
    const uint8_t* ab = p.a + (int64_t)kb * 128;
#pragma unroll
    for (int i = 0; i < 2; ++i) dma16(ab, P.aoff[i], st + (16 * wave + 8 * i) * 128);
    if constexpr (LO) {
      const uint8_t* al = p.a_lo + (int64_t)kb * 128;
#pragma unroll
      for (int i = 0; i < 2; ++i) dma16(al, P.aoff[i], st + F8_A_BYTES + (16 * wave + 8 * i) * 128);
    }
#pragma unroll
    for (int b2 = 0; b2 < BPW; ++b2) {
      const int b = wave * BPW + b2;
      dma16(P.bsrc[b2] + (int64_t)kb * 16384, lane * 16, st + F8_B_OFF + (b >> 1) * 2048 + (b & 1) * 1024);
    }
    if (has_sa) dma4(p.sa + kb, P.soff, st + F8_SA_OFF + (wave - 4) * 256);
    if (has_sw) dma4(P.swsrc + kb, 0u, st + F8_SW_OFF + (wave - 6) * 256);
  };

  // ---- MFMA side: lane (h, c32) = (lane >> 5, lane & 31) ----
  const int c32 = lane & 31, h = lane >> 5;
  const int fsw = f8_swz(c32);
  // A operand of k-step s (K = 64): row c32 of the 32-row tile, bytes
  // 64s + 32h .. +32 = pieces 4s + 2h and 4s + 2h + 1
  uint32_t adoff[2][2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int e = 0; e < 2; ++e) adoff[s][e] = (mw * 64 + c32) * 128 + (((4 * s + 2 * h + e) ^ fsw) * 16);
  // B operand: column c32 of the tile = column c32 & 15 of 16-column weight
  // tile (c32 >> 4); bytes 64s + 32h .. +32 are the two halves of the slot of
  // lane 16 * (2s + h) + (c32 & 15)
  uint32_t bdoff[C32][2];
  int swq[C32];
#pragma unroll
  for (int c = 0; c < C32; ++c) {
    const int q = c / CQ, cc = c - q * CQ;
    const int t16 = q * TPM + nw * CTW + 2 * cc + (c32 >> 4);
#pragma unroll
    for (int s = 0; s < 2; ++s) bdoff[c][s] = F8_B_OFF + t16 * 2048 + (16 * (2 * s + h) + (c32 & 15)) * 16;
    swq[c] = NQ == 2 ? q : (WGN == 256 ? nw >> 1 : 0);
  }

  f32x16 acc[2][C32];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int c = 0; c < C32; ++c) acc[rt][c] = f32x16{};

  auto compute = [&](int slot) {
    const char* S = smem + slot * F8_STAGE;
    float swv[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) swv[q] = *reinterpret_cast<const float*>(S + F8_SW_OFF + q * 256);
    f32x16 t[2][C32];
    // LO: the low parts first (part 0 at byte F8_A_BYTES), t /= 16, then the
    // high parts accumulate onto t
#pragma unroll
    for (int part = LO ? 0 : 1; part < 2; ++part) {
      const char* SA = S + (part == 0 ? F8_A_BYTES : 0);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        i32x8 a[2], b[C32];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          const u32x4 lo = *reinterpret_cast<const u32x4*>(SA + rt * 32 * 128 + adoff[s][0]);
          const u32x4 hi = *reinterpret_cast<const u32x4*>(SA + rt * 32 * 128 + adoff[s][1]);
          a[rt] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        }
#pragma unroll
        for (int c = 0; c < C32; ++c) {
          const u32x4 lo = *reinterpret_cast<const u32x4*>(S + bdoff[c][s]);
          const u32x4 hi = *reinterpret_cast<const u32x4*>(S + bdoff[c][s] + 1024);
          b[c] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        }
        const bool fresh = s == 0 && (LO ? part == 0 : true);
#pragma unroll
        for (int c = 0; c < C32; ++c)
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) t[rt][c] = mfma_f8_32(a[rt], b[c], fresh ? f32x16{} : t[rt][c]);
      }
      if (LO && part == 0) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
          for (int c = 0; c < C32; ++c)
#pragma unroll
            for (int i = 0; i < 16; ++i) t[rt][c][i] *= 0.0625f;
      }
    }
    // acc += (s_a[row] * s_w[block]) * t; register i of tile rt holds row
    // mw*64 + 32*rt + 8*(i/4) + 4*h + i%4
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 sa = *reinterpret_cast<const f32x4*>(S + F8_SA_OFF + (mw * 64 + 32 * rt + 8 * g + 4 * h) * 4);
#pragma unroll
        for (int c = 0; c < C32; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc[rt][c][4 * g + e] = fmaf(sa[e] * swv[swq[c]], t[rt][c][4 * g + e], acc[rt][c][4 * g + e]);
      }
  };

  auto row_of = [&](int rt, int i) { return mw * 64 + 32 * rt + 8 * (i >> 2) + 4 * h + (i & 3); };
  auto epilogue = [&](int j, const Plan& P) {
    const int* R = Rid[j % 3];
    if constexpr (EPI == F8_SILU_Q) {
      // h = silu(g) * u in float32, then high and low e4m3 parts per row
      // per 128-column block (this item's columns): scale = max(amax, 1e-12) / 448
      float hv[32], am[32];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float g = acc[rt][0][i], u = acc[rt][1][i];
          hv[rt * 16 + i] = g * __frcp_rn(1.0f + __expf(-g)) * u;
          am[rt * 16 + i] = fabsf(hv[rt * 16 + i]);
        }
      const float wmax = half_wave_row_reduce<true>(am, c32);
      part[nw * F8_BM + row_of(c32 >> 4, c32 & 15)] = wmax;
      lds_barrier();
      if (tid < F8_BM)
        amax_s[tid] = fmaxf(fmaxf(part[tid], part[F8_BM + tid]), fmaxf(part[2 * F8_BM + tid], part[3 * F8_BM + tid]));
      lds_barrier();
      const int64_t col = (int64_t)P.nb * WGN + nw * CTW * 16 + c32;
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 amx = *reinterpret_cast<const f32x4*>(&amax_s[mw * 64 + 32 * rt + 8 * g + 4 * h]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int row = row_of(rt, 4 * g + e);
            if (row < P.nvalid) {
              const float sc = fmaxf(amx[e], kAmaxFloor) / kFp8Max;
              const float v = hv[rt * 16 + 4 * g + e] / sc;
              const uint32_t qh = f32_to_fp8_rne(v);
              // v - fp8(qh) is exact (qh is v's nearest e4m3 value), and so is * 16
              const uint32_t ql = f32_to_fp8_rne((v - fp8_e4m3_to_f32(qh)) * 16.0f);
              p.qy[(int64_t)R[row] * p.ldqy + col] = (uint8_t)qh;
              p.qy_lo[(int64_t)R[row] * p.ldqy + col] = (uint8_t)ql;
            }
          }
        }
      if (tid < P.nvalid) p.sy[(int64_t)R[tid] * p.ldsy + P.nb] = fmaxf(amax_s[tid], kAmaxFloor) / kFp8Max;
    } else {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int row = row_of(rt, i);
          if (row >= P.nvalid) continue;
          const int64_t o = (int64_t)R[row] * p.ldy + P.nb * WGN + nw * CTW * 16 + c32;
#pragma unroll
          for (int c = 0; c < C32; ++c) {
            const float v = acc[rt][c][i];
            if (p.y_dtype == CCQ_F32)
              reinterpret_cast<float*>(p.y)[o + c * 32] = v;
            else if (p.y_dtype == CCQ_BF16)
              reinterpret_cast<uint16_t*>(p.y)[o + c * 32] = (uint16_t)f32_to_bf16_bits(v);
            else
              reinterpret_cast<uint16_t*>(p.y)[o + c * 32] = (uint16_t)f32_to_f16_bits(v);
          }
        }
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int c = 0; c < C32; ++c) acc[rt][c] = f32x16{};
  };

  // ---- pipeline over all K blocks of all items of this workgroup ----
  Plan cur, nxt;
  make_plan(0, cur);
  if (nmine > 1) make_plan(1, nxt);
  issue(cur, 0, 0);
  if (total > 1) issue(cur, 1, 1);  // KB >= 2
  int j = 0, kb = 0, slot = 0;
  for (int g = 0; g < total; ++g) {
    if (g + 1 < total)
      wait_stage<8>(ncopy);
    else
      wait_vmcnt<0>();
    lds_barrier();
    if (kb == 0 && j + 2 < nmine) fetch_rows(j + 2);
    if (kb == KB - 2 && j + 1 < nmine) make_plan(j + 1, nxt);
    const bool last = kb + 1 == KB;
    const int slot2 = slot == 0 ? 2 : slot - 1;  // (slot + 2) % 3
    if (!last && g + 2 < total) issue(kb + 2 < KB ? cur : nxt, kb + 2 < KB ? kb + 2 : kb + 2 - KB, slot2);
    if (mw * 64 < cur.nvalid) compute(slot);
    if (last) {
      epilogue(j, cur);
      if (g + 2 < total) issue(nxt, 1, slot2);
      cur = nxt;
      ++j;
      kb = 0;
    } else {
      ++kb;
    }
    slot = slot == 2 ? 0 : slot + 1;
  }
}

// ------------------------------------------ MoE stages, weights in VGPRs --
// The MoE stages (F8_SILU_Q gate/up, F8_ROWS down with the high and low
// intermediate parts) on the same persistent schedule, with the weights
// streamed straight into registers.  A workgroup is RB_NW waves; wave w
// owns RB_CG 32-column MFMA groups of every 128-row tile -- for gate/up,
// gate columns nb*128 + 16(RB_CG w + cg) + c and the same up columns
// (c = lane & 15, the up half in lanes 16..31); for down, columns
// nb*256 + 32(RB_CG w + cg) + (lane & 31) -- and loads their 16-byte
// weight slices itself, RB_D K blocks ahead (64 B per lane and K block:
// 96 KiB of weights in flight per compute unit at RB_D = 3).  Only the activation tiles and their scales go through LDS, in a
// ring of SA K blocks filled by LDS DMA; one barrier per K block.  Both the
// copies and the weight loads are inline assembly sharing the wave's
// in-order vmcnt (a compiler-issued load would be waited for by a count
// that ignores the copies issued after it, draining the pipeline), and the
// weight registers are handed to the compiler by a wait whose "+v" operands
// are those registers.  Every wave issues the same number of memory
// operations per K block (waves without a scale to copy copy one into a
// pad), so all waits are fixed vmcnt values; the first steps wait for
// more, and the steps past the end re-issue the last K block's loads so
// that the counts stay exact.  All four row tiles of an item are computed
// whatever its number of valid rows: MFMA time stays under the weight
// stream's time at 128 rows.
constexpr int RB_NW = 8;  // waves per workgroup
constexpr int RB_CG = 1;  // 32-column MFMA groups per wave
constexpr int RB_D = 3;   // K blocks of weight loads issued ahead per wave
static_assert(RB_NW * RB_CG == 8, "256 columns (down) / 2 x 128 (gate/up) per item");
static_assert(RB_CG == 1, "one register set of weight quads per K block and wait");

template <bool LO>
struct RbStage {
  static constexpr int NA = LO ? 2 : 1;                  // activation parts
  static constexpr int SA = LO ? 4 : 6;                  // activation ring stages
  static constexpr int RPW = F8_BM / RB_NW;              // activation rows copied per wave (8 per copy)
  static constexpr int A = F8_A_BYTES * NA;
  static constexpr int SA_OFF = A;                       // s_a of the 128 rows
  static constexpr int SW_OFF = SA_OFF + F8_BM * 4;      // 2 x 64 copies of a block scale
  static constexpr int PAD_OFF = SW_OFF + 2 * 256;       // the copies of waves 4.. (count padding)
  static constexpr int BYTES = PAD_OFF + (RB_NW > 4 ? (RB_NW - 4) * 256 : 0);
  static constexpr int NB = 4 * RB_CG;                   // weight loads per wave and K block
  static constexpr int A_OPS = NA * RPW / 8 + 1;        // activation + scale copies per wave and K block
  static constexpr int N_OPS = A_OPS + NB;               // memory operations per wave and K block
  // vmcnt allowed in steady state while waiting for the activation stage of
  // step g (copied at step g - SA + 1, followed by that step's weight loads
  // and SA - 2 whole steps)
  static constexpr int WAIT_A = NB + (SA - 2) * N_OPS;
  // vmcnt allowed while waiting for the weights of step g (loaded at step
  // g - RB_D, followed by RB_D - 1 whole steps; step g's copies are issued
  // after this wait; the prologue follows each of its weight loads by A_OPS
  // pad copies, so the count also holds, with room, from step 0)
  static constexpr int WAIT_B = (RB_D - 1) * N_OPS;
  static_assert(WAIT_A < 64 && WAIT_B < 64, "vmcnt is 6 bits");
};
template <bool LO>
constexpr size_t rb_lds_bytes() {
  return (size_t)RbStage<LO>::SA * RbStage<LO>::BYTES + 3 * F8_RID * 4 + (RB_NW + 1) * F8_BM * 4;
}
static_assert(rb_lds_bytes<true>() <= 160 * 1024 && rb_lds_bytes<false>() <= 160 * 1024, "LDS budget");

template <int EPI, bool LO>
__global__ __launch_bounds__(RB_NW * 64) void fp8_moe_rb_kernel(const Fp8GP p) {
  static_assert(EPI == F8_SILU_Q || EPI == F8_ROWS, "MoE stages");
  static_assert(!LO || EPI == F8_ROWS, "the low parts feed the down stage");
  using SL = RbStage<LO>;
  constexpr int NA = SL::NA, SA = SL::SA, D = RB_D, NW = RB_NW, CG = RB_CG, RPW = SL::RPW;
  constexpr int WGN = EPI == F8_SILU_Q ? 128 : 256;  // columns of each matrix per item
  __shared__ __align__(16) char smem[SA * SL::BYTES];
  __shared__ __align__(16) int Rid[3][F8_RID];
  __shared__ __align__(16) float part[NW * F8_BM];
  __shared__ __align__(16) float amax_s[F8_BM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c32 = lane & 31, h = lane >> 5;
  const int nblk = p.N / WGN;
  const int ntiles = p.meta != nullptr ? p.meta[0] : p.tiles;
  const int xcd = blockIdx.x & 7, wx = blockIdx.x >> 3;
  const int nx = ((int)gridDim.x - xcd + 7) >> 3;
  const int items_x = (ntiles > xcd ? (ntiles - xcd + 7) >> 3 : 0) * nblk;
  if (wx >= items_x) return;
  // rounds of nx items in alternating direction, as in the int4 kernel
  auto item_of = [&](int j) { return j * nx + ((j & 1) ? nx - 1 - wx : wx); };
  const int nmine = items_x / nx + (item_of(items_x / nx) < items_x ? 1 : 0);
  const int KB = p.KB;

  auto tile_of = [&](int j) { return xcd + 8 * (item_of(j) / nblk); };
  auto fetch_rows = [&](int j) {  // row ids of item j (+ its expert) into Rid[j % 3], by DMA
    if (j >= nmine) return;
    const int tile = tile_of(j);
    const uint32_t dst = lds_addr(&Rid[j % 3][0]);
    if (wave >= NW - 2) {
      // (lane offsets recomputed here, not kept live across the K loop)
      const uint32_t loff = (uint32_t)lane_id_here() * 4;
      dma4(p.rows + (int64_t)tile * F8_BM + (wave - (NW - 2)) * 64, loff, dst + (wave - (NW - 2)) * 256);
    }
    if (wave == NW - 3) dma4(p.tile_expert + tile, 0u, dst + F8_BM * 4);
  };
  for (int j = 0; j < 2 && j < nmine; ++j) {
    const int tile = tile_of(j);
    if (tid < F8_BM) Rid[j][tid] = p.rows[(int64_t)tile * F8_BM + tid];
    if (tid == F8_BM) Rid[j][F8_BM] = p.tile_expert[tile];
  }
  __syncthreads();

  // ---- per-item plan of this wave ----
  struct Plan {
    uint32_t aoff[RPW / 8];  // the activation rows this wave copies (8 per copy)
    uint32_t soff;           // waves 0, 1: their s_a rows
    const uint8_t* b;        // this lane's weight slices of MFMA group 0, K block 0
    const float* scsrc;      // waves 2, 3: the block scale copied
    int nvalid, nb;
  };
  auto make_plan = [&](int j, Plan& P) {
    // (lane values recomputed here, not kept live across the K loop)
    const int lane = lane_id_here(), c32 = lane & 31, h = lane >> 5;
    P.nb = item_of(j) % nblk;
    const int* R = Rid[j % 3];
    const int ex = __builtin_amdgcn_readfirstlane(R[F8_BM]);
    P.nvalid = (int)(__popcll(__ballot(R[lane] >= 0)) + __popcll(__ballot(R[64 + lane] >= 0)));
    const int rid0 = R[0];
#pragma unroll
    for (int i = 0; i < RPW / 8; ++i) {
      const int row = RPW * wave + 8 * i + (lane >> 3);
      const int rid = R[row] >= 0 ? R[row] : rid0;
      const int arow = EPI == F8_SILU_Q ? rid / p.row_div : rid;  // the down stage's rows are assignments
      P.aoff[i] = (uint32_t)((int64_t)arow * p.lda + ((lane & 7) ^ f8_swz(row)) * 16);
    }
    P.soff = 0;
    if (wave < 2) {
      const int row = 64 * wave + lane;
      const int rid = R[row] >= 0 ? R[row] : rid0;
      P.soff = (uint32_t)((int64_t)(EPI == F8_SILU_Q ? rid / p.row_div : rid) * p.ldsa * 4);
    }
    int64_t nt;  // the lane's 16-column weight tile
    const uint8_t* base = p.w0;
    if constexpr (EPI == F8_SILU_Q) {
      nt = (int64_t)P.nb * 8 + CG * wave;
      if (c32 >= 16) base = p.w1;
    } else {
      nt = (int64_t)P.nb * 16 + 2 * CG * wave + (c32 >> 4);
    }
    P.b = base + (int64_t)ex * p.w_es + fp8_chunk_off(nt, 0, KB) + (16 * h + (c32 & 15)) * 16;
    P.scsrc = nullptr;
    if (wave == 2 || wave == 3) {
      const int q = wave - 2;
      if constexpr (EPI == F8_SILU_Q)
        P.scsrc = (q == 0 ? p.sw0 : p.sw1) + (int64_t)ex * p.sw_es + (int64_t)P.nb * KB;
      else
        P.scsrc = p.sw0 + (int64_t)ex * p.sw_es + (int64_t)(2 * P.nb + q) * KB;
    }
  };
  Plan cur, nxt;
  const uint32_t lds0 = lds_addr(smem);
  // activation copies of K block kb of a plan into ring slot `slot`: NA x
  // RPW / 8 row copies + 1 scale copy per wave
  // (the plan is chosen by select, not by branch: every copy and load is
  // issued on one path, so no register of an in-flight load is merged
  // between branches)
  auto issue_a = [&](bool next, int kb, int slot) {
    const uint32_t st = lds0 + slot * SL::BYTES;
    const uint8_t* ab = p.a + (int64_t)kb * 128;
    uint32_t aoff[RPW / 8];
#pragma unroll
    for (int i = 0; i < RPW / 8; ++i) aoff[i] = next ? nxt.aoff[i] : cur.aoff[i];
#pragma unroll
    for (int i = 0; i < RPW / 8; ++i) dma16(ab, aoff[i], st + (RPW * wave + 8 * i) * 128);
    if constexpr (LO) {
      const uint8_t* al = p.a_lo + (int64_t)kb * 128;
#pragma unroll
      for (int i = 0; i < RPW / 8; ++i) dma16(al, aoff[i], st + F8_A_BYTES + (RPW * wave + 8 * i) * 128);
    }
    // one scale copy per wave, chosen by wave-uniform selects: the s_a rows
    // (waves 0, 1), a block scale (waves 2, 3) or a pad copy
    const float* src = wave >= 2 && wave < 4 ? (next ? nxt.scsrc : cur.scsrc) : p.sa;
    const uint32_t voff = wave < 2 ? (next ? nxt.soff : cur.soff) : 0u;
    const uint32_t dst = wave < 2 ? SL::SA_OFF + wave * 256
                                  : (wave < 4 ? SL::SW_OFF + (wave - 2) * 256 : SL::PAD_OFF + (wave - 4) * 256);
    dma4(src + kb, voff, st + dst);
  };
  // this lane's weight slices of K block kb: the B operands [k-step][half]
  // (bytes 0..15 and 16..31 of the lane's 32 are the two 1 KiB halves),
  // loaded by inline assembly and waited for with wait_vmcnt_tied
  auto issue_b = [&](bool next, int kb, u32x4 (&bq)[2][2]) {
    const uint8_t* b = (next ? nxt.b : cur.b) + (int64_t)kb * 16384;
    gload16_nt<0>(bq[0][0], b);
    gload16_nt<1024>(bq[0][1], b);
    gload16_nt<512>(bq[1][0], b);
    gload16_nt<1536>(bq[1][1], b);
  };

  // ---- MFMA side.  The weights are the A operand (MFMA rows = the wave's
  // 32 weight columns: gate/up, 16 gate columns then the same 16 up
  // columns) and the activations the B operand (MFMA columns = the 32 rows
  // of a row tile; lane (c32, h) holds row c32, pieces 4s + 2h, 4s + 2h + 1
  // of k-step s).  Register i of row tile rt then holds row 32 rt + c32 and
  // weight column 8 (i / 4) + 4 h + i % 4 of the wave's group: for gate/up,
  // i < 8 a gate column and i + 8 the same up column. ----
  const int fsw = f8_swz(c32);
  uint32_t adoff[2][2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int e = 0; e < 2; ++e) adoff[s][e] = c32 * 128 + (((4 * s + 2 * h + e) ^ fsw) * 16);
  // down: which of the two copied block scales (the 128-column block of the wave's columns)
  const int swq = (CG * wave) / 4;

  f32x16 acc[4][CG];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) acc[rt][cg] = f32x16{};

  // One K block over the row tiles holding valid rows (nrt = 1..4,
  // wave-uniform), software-pipelined: the MFMAs of row tile rt + 1 are
  // issued before the scaling of row tile rt, which then runs under them.
  // mid (the activation copies of a later step) runs after the first row
  // tile's MFMAs are issued, so that its scalar work overlaps them
  auto compute = [&](int slot, int nrt, const i32x8 (&bq)[CG][2], auto&& mid) {
    const char* S = smem + slot * SL::BYTES;
    // block scales of the wave's columns: gate (copy 0) and up (copy 1), or
    // the one block of the down columns
    const float sw0 = *reinterpret_cast<const float*>(S + SL::SW_OFF + (EPI == F8_SILU_Q ? 0 : swq * 256));
    const float sw1 = EPI == F8_SILU_Q ? *reinterpret_cast<const float*>(S + SL::SW_OFF + 256) : sw0;
    auto mma = [&](int rt) {
      f32x16 t;
      // LO: the low parts first, scaled by 1/16 inside the MFMA, then the
      // high parts accumulate onto them
#pragma unroll
      for (int part = LO ? 0 : 1; part < 2; ++part) {
        const char* ar = S + (part == 0 ? F8_A_BYTES : 0) + rt * 32 * 128;
        i32x8 a[2];
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const u32x4 lo = *reinterpret_cast<const u32x4*>(ar + adoff[st][0]);
          const u32x4 hi = *reinterpret_cast<const u32x4*>(ar + adoff[st][1]);
          a[st] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        }
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const bool fresh = st == 0 && (LO ? part == 0 : true);
          if (LO && part == 0)
            t = mfma_f8_32_b16th(bq[0][st], a[st], fresh ? f32x16{} : t);
          else
            t = mfma_f8_32(bq[0][st], a[st], fresh ? f32x16{} : t);
        }
      }
      return t;
    };
    // acc += (s_a[row] * s_w[column]) * t; the lane's row has one s_a
    auto scale = [&](int rt, const f32x16& t) {
      const float sa = *reinterpret_cast<const float*>(S + SL::SA_OFF + (32 * rt + c32) * 4);
      const float f0 = sa * sw0, f1 = sa * sw1;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[rt][0][i] = fmaf(i < 8 ? f0 : f1, t[i], acc[rt][0][i]);
    };
    f32x16 t = mma(0);
    mid();
#pragma unroll
    for (int rt = 1; rt < 4; ++rt) {
      if (rt < nrt) {
        const f32x16 tn = mma(rt);
        scale(rt - 1, t);
        t = tn;
      } else if (rt == nrt) {
        scale(rt - 1, t);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (nrt == 4) scale(3, t);
  };

  auto epilogue = [&](int j, const Plan& P) {
    const int* R = Rid[j % 3];
    if constexpr (EPI == F8_SILU_Q) {
      // h = silu(gate) * up in float32 in the lane (registers i, i + 8).  Row
      // amax over the item's 128 columns: the lane's 8, the lane holding the
      // row's other 8 columns of the wave (h ^ 1), then the waves via LDS.
      // Row tiles without valid rows are skipped (wave-uniform).
      const int nrt = (P.nvalid + 31) >> 5;
      float hq[4][8];
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        if (rt < nrt) {
          float am = 0.f;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float g = acc[rt][0][i], u = acc[rt][0][i + 8];
            const float hv = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
            hq[rt][i] = hv;
            am = fmaxf(am, fabsf(hv));
          }
          am = fmaxf(am, __shfl_xor(am, 32, 64));
          if (h == 0) part[wave * F8_BM + 32 * rt + c32] = am;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      lds_barrier();
      if (tid < 32 * nrt) {
        float mx = part[tid];
#pragma unroll
        for (int w = 1; w < NW; ++w) mx = fmaxf(mx, part[w * F8_BM + tid]);
        amax_s[tid] = mx;
      }
      lds_barrier();
      // columns 8q + 4h .. + 3 of the wave's 16: four bytes per store.  The
      // e4m3 conversions are the hardware's (v_cvt_pk_fp8_f32, round to
      // nearest even; equal to the software encoder for every |v| <= 460,
      // and |v| <= 448 (1 + 2^-22) here).
      const int64_t col0 = (int64_t)P.nb * WGN + 16 * (CG * wave) + 4 * h;
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const int row = 32 * rt + c32;
        if (rt < nrt && row < P.nvalid) {
          const float am = fmaxf(amax_s[row], kAmaxFloor);
          const float inv = kFp8Max / am;  // v = h / (am / 448) up to an ulp
          const int64_t o = (int64_t)R[row] * p.ldqy + col0;
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = hq[rt][4 * q + e] * inv;
            int wh = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
            wh = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], wh, true);
            // v - fp8(hi) is exact (hi is v's nearest e4m3 value), and so is * 16
            const auto b01 = __builtin_amdgcn_cvt_pk_f32_fp8(wh, false);
            const auto b23 = __builtin_amdgcn_cvt_pk_f32_fp8(wh, true);
            int wl = __builtin_amdgcn_cvt_pk_fp8_f32((v[0] - b01[0]) * 16.0f, (v[1] - b01[1]) * 16.0f, 0, false);
            wl = __builtin_amdgcn_cvt_pk_fp8_f32((v[2] - b23[0]) * 16.0f, (v[3] - b23[1]) * 16.0f, wl, true);
            *reinterpret_cast<uint32_t*>(p.qy + o + 8 * q) = (uint32_t)wh;
            *reinterpret_cast<uint32_t*>(p.qy_lo + o + 8 * q) = (uint32_t)wl;
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (tid < P.nvalid) p.sy[(int64_t)R[tid] * p.ldsy + P.nb] = fmaxf(amax_s[tid], kAmaxFloor) / kFp8Max;
    } else {
      // columns 8q + 4h .. + 3 of the wave's 32: four values per store
      const int64_t col0 = (int64_t)P.nb * WGN + 32 * (CG * wave) + 4 * h;
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const int row = 32 * rt + c32;
        if (row < P.nvalid) {
          const int64_t o = (int64_t)R[row] * p.ldy + col0;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x16& v = acc[rt][0];
            if (p.y_dtype == CCQ_F32) {
              *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p.y) + o + 8 * q) =
                  f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
            } else {
              const bool bf = p.y_dtype == CCQ_BF16;
              uint32_t w2[2];
#pragma unroll
              for (int e = 0; e < 2; ++e) {
                const float x0 = v[4 * q + 2 * e], x1 = v[4 * q + 2 * e + 1];
                w2[e] = bf ? (f32_to_bf16_bits(x0) | (f32_to_bf16_bits(x1) << 16))
                           : (f32_to_f16_bits(x0) | (f32_to_f16_bits(x1) << 16));
              }
              *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.y) + o + 8 * q) = u32x2{w2[0], w2[1]};
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) acc[rt][cg] = f32x16{};
  };

  // ---- the pipeline over all K blocks of all items of this workgroup.  Step
  // g: wait for its activation stage, barrier, copy the activations of step
  // g + SA - 1 into the slot step g - 1 used, wait for its weights, compute,
  // load the weights of step g + D into the registers just used.  Steps past
  // the end re-issue the last step's loads (same counts).  `cur` is the
  // plan of the current item, `nxt` that of the next one. ----
  make_plan(0, cur);
  nxt = cur;
  if (nmine > 1) make_plan(1, nxt);
  // (next item?, kb) of the step `ahead` steps after (j, kb), ahead < KB,
  // clamped to the last step
  auto ahead_of = [&](int j, int kb, int ahead, bool& next, int& pk) {
    int k2 = kb + ahead, j2 = j;
    if (k2 >= KB) {
      k2 -= KB;
      ++j2;
    }
    if (j2 >= nmine) {
      j2 = nmine - 1;
      k2 = KB - 1;
    }
    next = j2 != j;
    pk = k2;
  };
#pragma unroll
  for (int g = 0; g < SA - 1; ++g) {
    bool nx_;
    int pk;
    ahead_of(0, 0, g, nx_, pk);
    issue_a(nx_, pk, g);
  }
  u32x4 bq[D][2][2];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    bool nx_;
    int pk;
    ahead_of(0, 0, d, nx_, pk);
    issue_b(nx_, pk, bq[d]);
#pragma unroll
    for (int i = 0; i < SL::A_OPS; ++i) dma4(p.sa, 0u, lds0 + SL::PAD_OFF + (wave & 3) * 256);
  }
  const int total = nmine * KB;
  int slot = 0, j = 0, kb = 0;
  for (int g0 = 0; g0 < total; g0 += D) {  // step g uses register set g % D
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int g = g0 + d;
      if (g >= total) break;
      if (g >= SA - 1)
        wait_vmcnt<SL::WAIT_A>();
      else
        wait_vmcnt<0>();
      lds_barrier();
      if (kb == 0) {
        if (j + 2 < nmine) fetch_rows(j + 2);
        if (j > 0 && j + 1 < nmine) make_plan(j + 1, nxt);
      }
      // the activation copies of step g + SA - 1 go into the slot step g - 1
      // used (free after the barrier), issued inside the compute after this
      // step's weight wait; every step issues them, so the per-step order of
      // memory operations (copies, then weight loads) is unchanged
      auto copy_ahead = [&]() {
        bool nx_;
        int pk;
        ahead_of(j, kb, SA - 1, nx_, pk);
        issue_a(nx_, pk, slot == 0 ? SA - 1 : slot - 1);
      };
      wait_vmcnt_tied<SL::WAIT_B>(bq[d][0][0], bq[d][0][1], bq[d][1][0], bq[d][1][1]);
      {
        i32x8 bw[CG][2];
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const u32x4 lo = bq[d][st][0], hi = bq[d][st][1];
          bw[0][st] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        }
        compute(slot, (cur.nvalid + 31) >> 5, bw, copy_ahead);
      }
      {
        bool nx_;
        int pk;
        ahead_of(j, kb, D, nx_, pk);
        issue_b(nx_, pk, bq[d]);
      }
      slot = slot + 1 == SA ? 0 : slot + 1;
      __builtin_amdgcn_sched_barrier(0);  // one step at a time
      if (kb + 1 == KB) {
        epilogue(j, cur);
        cur = nxt;
        ++j;
        kb = 0;
        __builtin_amdgcn_sched_barrier(0);
      } else {
        ++kb;
      }
    }
  }
  // no copy into LDS outlives the workgroup, and the registers of the last
  // (unused) weight loads stay reserved until they have landed
#pragma unroll
  for (int d = 0; d < D; ++d) wait_vmcnt_tied<0>(bq[d][0][0], bq[d][0][1], bq[d][1][0], bq[d][1][1]);
}

// Compute units of the current device (one persistent workgroup each; at
// least 8 so that every XCD gets one).
static int f8_device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n < 8 ? 8 : n;
  }
  return cus[dev];
}

// tiles = 128-row schedule tiles the grid is sized for (the kernel reads the
// actual number from meta when given).  K must hold at least 2 blocks.
// The MoE stages with the weights in registers need K blocks of lookahead
// inside one item plus the next (KB >= 6), a schedule (rows, experts) and
// outputs aligned for their vector stores (4 columns per store).
static bool use_rb(const Fp8GP& p, bool silu) {
  if (p.KB < 6 || p.rows == nullptr || p.tile_expert == nullptr) return false;
  if (silu)
    return p.ldqy % 4 == 0 && ((uintptr_t)p.qy & 3) == 0 && ((uintptr_t)p.qy_lo & 3) == 0;
  const uintptr_t al = p.y_dtype == CCQ_F32 ? 15 : 7;
  return p.ldy % 4 == 0 && ((uintptr_t)p.y & al) == 0;
}

template <int EPI>
static int launch_fp8_gemm(const Fp8GP& p, int64_t tiles, hipStream_t st) {
  const bool lo = p.a_lo != nullptr;
  if constexpr (EPI != F8_STORE) {
    if (use_rb(p, EPI == F8_SILU_Q)) {
      const int wgn = EPI == F8_SILU_Q ? 128 : 256;
      if (p.N % wgn == 0) {
        const int64_t items = tiles * (p.N / wgn), cus = f8_device_cus();
        const dim3 grid((unsigned)(items < cus ? items : cus)), block(RB_NW * 64);
        if constexpr (EPI == F8_SILU_Q)
          launch((fp8_moe_rb_kernel<F8_SILU_Q, false>), grid, block, 0, st, p);
        else if (lo)
          launch((fp8_moe_rb_kernel<F8_ROWS, true>), grid, block, 0, st, p);
        else
          launch((fp8_moe_rb_kernel<F8_ROWS, false>), grid, block, 0, st, p);
        return launch_status("fp8 moe gemm");
      }
    }
  }
  if (lo && EPI != F8_ROWS) return arg_error("fp8 gemm: low activation parts need the row epilogue");
  // the high + low activation tiles take the LDS of half the weight tiles
  const int wgn = EPI == F8_SILU_Q || lo ? 128 : (p.N % 256 == 0 ? 256 : 128);
  const int64_t items = tiles * (p.N / wgn), cus = f8_device_cus();
  const dim3 grid((unsigned)(items < cus ? items : cus)), block(512);
  if constexpr (EPI == F8_ROWS) {
    if (lo) {
      launch((fp8_gemm_kernel<EPI, 2, true>), grid, block, 0, st, p);
      return launch_status("fp8 gemm");
    }
  }
  if (wgn == 256)
    launch((fp8_gemm_kernel<EPI, (EPI == F8_SILU_Q ? 2 : 4)>), grid, block, 0, st, p);
  else
    launch((fp8_gemm_kernel<EPI, 2>), grid, block, 0, st, p);
  return launch_status("fp8 gemm");
}

static int grid_of(int64_t n, int block) {
  const int64_t g = cdiv(n, block);
  return (int)(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

int launch_act_quant(const void* x, int x_dtype, int64_t ldx, int64_t rows, int64_t K, uint8_t* q, int64_t ldq,
                     float* s, int64_t lds_, hipStream_t st) {
  const int64_t KB = K / 128;
  if (rows * KB >= (1LL << 31)) return arg_error("fp8 act quant: %lld rows x K/128=%lld too large", (long long)rows, (long long)KB);
  const dim3 grid(grid_of(rows * KB * 16, 256));
  if (aligned(x, 16) && ldx % (x_dtype == CCQ_F32 ? 4 : 8) == 0) {
    if (x_dtype == CCQ_BF16)
      launch(fp8_act_quant_vec_kernel<CCQ_BF16>, grid, dim3(256), 0, st, x, ldx, q, ldq, s, lds_, rows, KB);
    else if (x_dtype == CCQ_F16)
      launch(fp8_act_quant_vec_kernel<CCQ_F16>, grid, dim3(256), 0, st, x, ldx, q, ldq, s, lds_, rows, KB);
    else
      launch(fp8_act_quant_vec_kernel<CCQ_F32>, grid, dim3(256), 0, st, x, ldx, q, ldq, s, lds_, rows, KB);
    return launch_status("fp8 act quant");
  }
  if (x_dtype == CCQ_BF16)
    launch(fp8_act_quant_kernel<CCQ_BF16>, grid, dim3(256), 0, st, x, ldx, q, ldq, s, lds_, rows, KB);
  else if (x_dtype == CCQ_F16)
    launch(fp8_act_quant_kernel<CCQ_F16>, grid, dim3(256), 0, st, x, ldx, q, ldq, s, lds_, rows, KB);
  else
    launch(fp8_act_quant_kernel<CCQ_F32>, grid, dim3(256), 0, st, x, ldx, q, ldq, s, lds_, rows, KB);
  return launch_status("fp8 act quant");
}

}  // namespace ccq

using namespace ccq;

extern "C" int ccq_fp8_act_quant(const void* x, int x_dtype, int64_t rows, int64_t K, uint8_t* q, float* s,
                                 void* stream) {
  CCQ_REQUIRE(rows >= 0 && K >= 0, "ccq_fp8_act_quant: negative shape");
  CCQ_REQUIRE(K % 128 == 0, "ccq_fp8_act_quant: K=%lld not a multiple of 128", (long long)K);
  CCQ_REQUIRE(x_dtype == CCQ_F32 || x_dtype == CCQ_F16 || x_dtype == CCQ_BF16, "ccq_fp8_act_quant: bad x_dtype");
  if (rows == 0 || K == 0) return 0;
  CCQ_REQUIRE(x && q && s, "ccq_fp8_act_quant: null pointer");
  CCQ_REQUIRE(aligned(q, 8), "ccq_fp8_act_quant: q must be 8-byte aligned");
  return launch_act_quant(x, x_dtype, K, rows, K, q, K, s, K / 128, as_stream(stream));
}

extern "C" int ccq_fp8_block_repack(const uint8_t* w, uint8_t* tiled, int64_t N, int64_t K, void* stream) {
  CCQ_REQUIRE(N >= 0 && K >= 0, "ccq_fp8_block_repack: negative shape");
  CCQ_REQUIRE(N % 128 == 0 && K % 128 == 0, "ccq_fp8_block_repack: need N %% 128 == 0 and K %% 128 == 0");
  if (N == 0 || K == 0) return 0;
  CCQ_REQUIRE(w && tiled, "ccq_fp8_block_repack: null pointer");
  CCQ_REQUIRE(w != tiled, "ccq_fp8_block_repack: in-place is not supported");
  CCQ_REQUIRE(aligned(w, 16) && aligned(tiled, 16), "ccq_fp8_block_repack: pointers must be 16-byte aligned");
  launch(fp8_repack_kernel, dim3(grid_of(N * K / 16, 256)), dim3(256), 0, as_stream(stream), w, tiled,
                     N, K);
  return launch_status("ccq_fp8_block_repack");
}

extern "C" int ccq_fp8_block_unpack(const uint8_t* tiled, uint8_t* w, int64_t N, int64_t K, void* stream) {
  CCQ_REQUIRE(N >= 0 && K >= 0, "ccq_fp8_block_unpack: negative shape");
  CCQ_REQUIRE(N % 128 == 0 && K % 128 == 0, "ccq_fp8_block_unpack: need N %% 128 == 0 and K %% 128 == 0");
  if (N == 0 || K == 0) return 0;
  CCQ_REQUIRE(w && tiled, "ccq_fp8_block_unpack: null pointer");
  CCQ_REQUIRE(w != tiled, "ccq_fp8_block_unpack: in-place is not supported");
  CCQ_REQUIRE(aligned(w, 16) && aligned(tiled, 16), "ccq_fp8_block_unpack: pointers must be 16-byte aligned");
  launch(fp8_unpack_kernel, dim3(grid_of(N * K / 16, 256)), dim3(256), 0, as_stream(stream), tiled, w,
                     N, K);
  return launch_status("ccq_fp8_block_unpack");
}

extern "C" int ccq_fp8_block_dequant(const uint8_t* w, const float* s_w, float* out, int64_t N, int64_t K,
                                     void* stream) {
  CCQ_REQUIRE(N >= 0 && K >= 0, "ccq_fp8_block_dequant: negative shape");
  CCQ_REQUIRE(N == 0 || K <= INT64_MAX / N, "ccq_fp8_block_dequant: N*K overflows");
  if (N == 0 || K == 0) return 0;
  CCQ_REQUIRE(w && s_w && out, "ccq_fp8_block_dequant: null pointer");
  launch(fp8_block_dequant_kernel, dim3(grid_of(N * K, 256)), dim3(256), 0, as_stream(stream), w, s_w,
                     out, N, K);
  return launch_status("ccq_fp8_block_dequant");
}

namespace {
size_t a256(size_t b) { return (b + 255) & ~(size_t)255; }

struct LinLayout {
  size_t off_q, off_s, total;
};
LinLayout lin_layout(int64_t M, int64_t K) {
  LinLayout L;
  size_t o = 0;
  L.off_q = o;
  o += a256((size_t)M * K);
  L.off_s = o;
  o += a256((size_t)M * (K / 128) * 4);
  L.total = o;
  return L;
}
}  // namespace

extern "C" size_t ccq_fp8_block_linear_workspace_size(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0 || K % 128) return 0;
  return lin_layout(M, K).total;
}

extern "C" int ccq_fp8_block_linear(const void* x, int x_dtype, const uint8_t* w_tiled, const float* s_w, void* y,
                                    int y_dtype, int64_t M, int64_t K, int64_t N, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  CCQ_REQUIRE(M >= 0 && K >= 0 && N >= 0, "ccq_fp8_block_linear: negative shape");
  CCQ_REQUIRE(K % 128 == 0 && N % 128 == 0, "ccq_fp8_block_linear: need K %% 128 == 0 and N %% 128 == 0 (K=%lld N=%lld)",
              (long long)K, (long long)N);
  CCQ_REQUIRE(x_dtype == CCQ_F32 || x_dtype == CCQ_F16 || x_dtype == CCQ_BF16, "ccq_fp8_block_linear: bad x_dtype");
  CCQ_REQUIRE(y_dtype == CCQ_F32 || y_dtype == CCQ_F16 || y_dtype == CCQ_BF16, "ccq_fp8_block_linear: bad y_dtype");
  CCQ_REQUIRE(cdiv(M, F8_BM) * (N / 128) <= 0x7fffffff, "ccq_fp8_block_linear: M or N too large");
  CCQ_REQUIRE(K == 0 || K >= 256, "ccq_fp8_block_linear: K=%lld < 256 (the kernel pipelines two 128-blocks)",
              (long long)K);
  CCQ_REQUIRE(M * K < (int64_t)1 << 32, "ccq_fp8_block_linear: activations of %lld x %lld exceed 4 GiB",
              (long long)M, (long long)K);
  if (M == 0 || N == 0) return 0;
  CCQ_REQUIRE(K > 0, "ccq_fp8_block_linear: K == 0");
  CCQ_REQUIRE(x && w_tiled && s_w && y, "ccq_fp8_block_linear: null pointer");
  CCQ_REQUIRE(aligned(w_tiled, 16), "ccq_fp8_block_linear: w_tiled must be 16-byte aligned");
  const LinLayout L = lin_layout(M, K);
  CCQ_REQUIRE(workspace && workspace_bytes >= L.total && aligned(workspace, 256),
              "ccq_fp8_block_linear: workspace of %zu bytes (256-byte aligned) needed, %zu given", L.total,
              workspace_bytes);
  hipStream_t st = as_stream(stream);
  uint8_t* q = (uint8_t*)workspace + L.off_q;
  float* s = (float*)((char*)workspace + L.off_s);
  int rc = launch_act_quant(x, x_dtype, K, M, K, q, K, s, K / 128, st);
  if (rc) return rc;
  Fp8GP p = {};
  p.a = q;
  p.lda = K;
  p.sa = s;
  p.ldsa = K / 128;
  p.row_div = 1;
  p.w0 = w_tiled;
  p.sw0 = s_w;
  p.y = y;
  p.ldy = N;
  p.y_dtype = y_dtype;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.KB = (int)(K / 128);
  p.tiles = (int)cdiv(M, F8_BM);
  return launch_fp8_gemm<F8_STORE>(p, p.tiles, st);
}

// ------------------------------------------------------------ MoE FP8 --
namespace {

int check_fp8_experts(const ccq_fp8_experts* ex, const char* name) {
  CCQ_REQUIRE(ex != nullptr, "%s: null expert descriptor", name);
  CCQ_REQUIRE(ex->num_experts >= 1 && ex->num_experts <= 1024, "%s: num_experts=%lld outside [1, 1024]", name,
              (long long)ex->num_experts);
  CCQ_REQUIRE(ex->hidden > 0 && ex->inter > 0 && ex->hidden % 128 == 0 && ex->inter % 128 == 0,
              "%s: hidden=%lld and inter=%lld must be positive multiples of 128", name, (long long)ex->hidden,
              (long long)ex->inter);
  CCQ_REQUIRE(ex->hidden <= (1 << 20) && ex->inter <= (1 << 20), "%s: hidden/inter too large", name);
  CCQ_REQUIRE(ex->hidden >= 256 && ex->inter >= 256,
              "%s: hidden=%lld and inter=%lld must be at least 256 (two 128-blocks)", name, (long long)ex->hidden,
              (long long)ex->inter);
  CCQ_REQUIRE(ex->w_gate && ex->s_gate && ex->w_up && ex->s_up && ex->w_down && ex->s_down,
              "%s: null weight pointer", name);
  CCQ_REQUIRE(aligned(ex->w_gate, 16) && aligned(ex->w_up, 16) && aligned(ex->w_down, 16),
              "%s: tiled weights must be 16-byte aligned", name);
  return 0;
}

struct F8MoeLayout {
  int64_t n, max_tiles;
  int bm;
  size_t off_sorted, off_te, off_meta, off_counts, off_qx, off_sx, off_qh, off_qh_lo, off_sh, off_rows, off_align,
      total;
};

F8MoeLayout f8_moe_layout(int64_t T, int64_t k, const ccq_fp8_experts* ex) {
  F8MoeLayout L;
  const int64_t H = ex->hidden, I = ex->inter;
  L.n = T * k;
  L.bm = F8_BM;
  L.max_tiles = ccq_moe_align_max_tiles(L.n, ex->num_experts, L.bm);
  size_t o = 0;
  L.off_sorted = o;
  o += a256((size_t)L.max_tiles * L.bm * 4);
  L.off_te = o;
  o += a256((size_t)L.max_tiles * 4);
  L.off_meta = o;
  o += 256;
  L.off_counts = o;
  o += a256((size_t)ex->num_experts * 4);
  L.off_qx = o;
  o += a256((size_t)T * H);
  L.off_sx = o;
  o += a256((size_t)T * (H / 128) * 4);
  L.off_qh = o;
  o += a256((size_t)L.n * I);
  L.off_qh_lo = o;
  o += a256((size_t)L.n * I);
  L.off_sh = o;
  o += a256((size_t)L.n * (I / 128) * 4);
  L.off_rows = o;
  o += a256((size_t)L.n * H * 4);
  L.off_align = o;  // per-chunk tables of the schedule of large batches
  o += a256(align_scratch_bytes(L.n, ex->num_experts));
  L.total = o;
  return L;
}

}  // namespace

extern "C" size_t ccq_moe_fp8_workspace_size(int64_t T, int64_t k, const ccq_fp8_experts* ex) {
  if (T <= 0 || k <= 0 || check_fp8_experts(ex, "ccq_moe_fp8_workspace_size") != 0) return 0;
  return f8_moe_layout(T, k, ex).total;
}

static int moe_fp8_ffn(const void* x, int x_dtype, const int64_t* ids, const float* weights, void* y, int y_dtype,
                       int64_t T, int64_t k, const ccq_fp8_experts* ex, void* workspace, size_t workspace_bytes,
                       void* stream, const float* shared, float shared_gate);

extern "C" int ccq_moe_fp8_ffn(const void* x, int x_dtype, const int64_t* ids, const float* weights, void* y,
                               int y_dtype, int64_t T, int64_t k, const ccq_fp8_experts* ex, void* workspace,
                               size_t workspace_bytes, void* stream) {
  return moe_fp8_ffn(x, x_dtype, ids, weights, y, y_dtype, T, k, ex, workspace, workspace_bytes, stream, nullptr,
                     0.f);
}

extern "C" int ccq_moe_fp8_ffn_shared(const void* x, int x_dtype, const int64_t* ids, const float* weights,
                                      const float* shared, float shared_gate, void* y, int y_dtype, int64_t T,
                                      int64_t k, const ccq_fp8_experts* ex, void* workspace, size_t workspace_bytes,
                                      void* stream) {
  CCQ_REQUIRE(shared || T == 0, "ccq_moe_fp8_ffn_shared: null shared");
  return moe_fp8_ffn(x, x_dtype, ids, weights, y, y_dtype, T, k, ex, workspace, workspace_bytes, stream, shared,
                     shared_gate);
}

static int moe_fp8_ffn(const void* x, int x_dtype, const int64_t* ids, const float* weights, void* y, int y_dtype,
                       int64_t T, int64_t k, const ccq_fp8_experts* ex, void* workspace, size_t workspace_bytes,
                       void* stream, const float* shared, float shared_gate) {
  int rc = check_fp8_experts(ex, "ccq_moe_fp8_ffn");
  if (rc) return rc;
  CCQ_REQUIRE(T >= 0 && k >= 1 && k <= ex->num_experts, "ccq_moe_fp8_ffn: bad T=%lld / k=%lld", (long long)T,
              (long long)k);
  CCQ_REQUIRE(T * k <= 65536, "ccq_moe_fp8_ffn: T*k=%lld > 65536", (long long)(T * k));
  CCQ_REQUIRE(T <= 65535, "ccq_moe_fp8_ffn: T=%lld > 65535", (long long)T);
  CCQ_REQUIRE(x_dtype == CCQ_F32 || x_dtype == CCQ_F16 || x_dtype == CCQ_BF16, "ccq_moe_fp8_ffn: bad x_dtype");
  CCQ_REQUIRE(y_dtype == CCQ_F32 || y_dtype == CCQ_F16 || y_dtype == CCQ_BF16, "ccq_moe_fp8_ffn: bad y_dtype");
  if (T == 0) return 0;
  CCQ_REQUIRE(x && ids && weights && y, "ccq_moe_fp8_ffn: null pointer");
  const F8MoeLayout L = f8_moe_layout(T, k, ex);
  CCQ_REQUIRE(T * ex->hidden < (int64_t)1 << 32 && L.n * ex->inter < (int64_t)1 << 32,
              "ccq_moe_fp8_ffn: activations exceed 4 GiB");
  CCQ_REQUIRE(workspace && workspace_bytes >= L.total && aligned(workspace, 256),
              "ccq_moe_fp8_ffn: workspace of %zu bytes (256-byte aligned) needed, %zu given", L.total,
              workspace_bytes);
  const int64_t H = ex->hidden, I = ex->inter;
  hipStream_t st = as_stream(stream);
  char* ws = (char*)workspace;
  int32_t* sorted = (int32_t*)(ws + L.off_sorted);
  int32_t* te = (int32_t*)(ws + L.off_te);
  int32_t* meta = (int32_t*)(ws + L.off_meta);
  int32_t* counts = (int32_t*)(ws + L.off_counts);
  uint8_t* qx = (uint8_t*)(ws + L.off_qx);
  float* sx = (float*)(ws + L.off_sx);
  uint8_t* qh = (uint8_t*)(ws + L.off_qh);
  uint8_t* qh_lo = (uint8_t*)(ws + L.off_qh_lo);
  float* sh = (float*)(ws + L.off_sh);
  void* rows = ws + L.off_rows;

  rc = launch_align(ids, L.n, ex->num_experts, L.bm, sorted, te, meta, counts, st, ws + L.off_align,
                    L.total - L.off_align);
  if (rc) return rc;
  rc = launch_act_quant(x, x_dtype, H, T, H, qx, H, sx, H / 128, st);
  if (rc) return rc;

  Fp8GP g = {};
  g.a = qx;
  g.lda = H;
  g.sa = sx;
  g.ldsa = H / 128;
  g.rows = sorted;
  g.row_div = (int)k;
  g.tile_expert = te;
  g.meta = meta;
  g.w0 = ex->w_gate;
  g.sw0 = ex->s_gate;
  g.w1 = ex->w_up;
  g.sw1 = ex->s_up;
  g.w_es = I * H;
  g.sw_es = (I / 128) * (H / 128);
  g.qy = qh;
  g.qy_lo = qh_lo;
  g.sy = sh;
  g.ldqy = I;
  g.ldsy = I / 128;
  g.N = (int)I;
  g.K = (int)H;
  g.KB = (int)(H / 128);
  rc = launch_fp8_gemm<F8_SILU_Q>(g, L.max_tiles, st);
  if (rc) return rc;

  Fp8GP d = {};
  d.a = qh;
  d.a_lo = qh_lo;
  d.lda = I;
  d.sa = sh;
  d.ldsa = I / 128;
  d.rows = sorted;
  d.row_div = 1;
  d.tile_expert = te;
  d.meta = meta;
  d.w0 = ex->w_down;
  d.sw0 = ex->s_down;
  d.w_es = H * I;
  d.sw_es = (H / 128) * (I / 128);
  d.y = rows;
  d.ldy = H;
  d.y_dtype = CCQ_BF16;  // bf16 rows: half the traffic of the row write and of the combine
  d.N = (int)H;
  d.K = (int)I;
  d.KB = (int)(I / 128);
  rc = launch_fp8_gemm<F8_ROWS>(d, L.max_tiles, st);
  if (rc) return rc;
  return launch_combine(rows, CCQ_BF16, weights, ids, ex->num_experts, y, y_dtype, T, k, H, st, shared,
                        shared_gate);
}
