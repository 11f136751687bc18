// FP8 e4m3fn with 128x128 block weight scales and per-token-per-128 dynamic
// activation scales on gfx950: activation quantization, weight re-pack, the
// block-scaled grouped GEMM on v_mfma_f32_16x16x128_f8f6f4, and the MoE
// expert FFN built on it.
//
// Format (public DeepSeek-V3-style block FP8): weights w [N, K] e4m3fn bytes
// (row = output channel) with s_w [N/128, K/128] float32,
// W[n, k] = fp8(w[n, k]) * s_w[n/128, k/128]; activations x [T, K] quantized
// per token per 128 channels: s_a = max(amax, 1e-12) / 448 (float32),
// q = RNE(x / s_a) saturated to +-448.  One 16x16x128 MFMA covers exactly one
// 128-wide K block, so each block's product is scaled once on the
// accumulator: acc += (s_a[row, kb] * s_w[nb, kb]) * mfma(q_a, q_w).
//
// Weight tile layout: tile (nt, kb) = 16 output channels x 128 K bytes =
// 2 KiB at byte (nt*KB + kb)*2048 (each wave streams one contiguous run of
// its 16 channels); inside, [half h][lane l][16 bytes] with
// bytes k = kb*128 + 32*(l >> 4) + 16*h + e of channel nt*16 + (l & 15).  A
// lane's 32 operand bytes (channel l & 15, K bytes 32*(l >> 4) .. +32) come
// from two wave-wide 16-byte loads, each a contiguous 1 KiB transfer.  The
// activation A operand uses the same K mapping (row l & 15, K bytes
// 32*(l >> 4) .. +32), so every K index meets its partner.
#include "ccq_common.h"

#include <math.h>

namespace ccq {

int launch_align(const int64_t* ids, int64_t n, int64_t E, int64_t tile_m, int32_t* sorted_ids,
                 int32_t* tile_expert, int32_t* meta, int32_t* counts, hipStream_t st);
int launch_combine(const void* rows, int rows_dtype, const float* wts, const int64_t* ids, int64_t E, void* y,
                   int y_dtype, int64_t T, int64_t k, int64_t H, hipStream_t st);

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
    const int64_t row = b / KB, kb = b - row * KB;
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

// ----------------------------------------------------------- re-pack --
// One thread per 16-byte piece of the tiled layout (a contiguous 16 bytes of
// one row of w).
__global__ void fp8_repack_kernel(const uint8_t* __restrict__ w, uint8_t* __restrict__ tiled, int64_t N,
                                  int64_t K) {
  const int64_t KB = K / 128, pieces = N * K / 16;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pieces;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int l = (int)(i & 63), h = (int)((i >> 6) & 1);
    const int64_t tile = i >> 7, kb = tile % KB, nt = tile / KB;
    const int64_t n = nt * 16 + (l & 15), k = kb * 128 + 32 * (l >> 4) + 16 * h;
    *reinterpret_cast<u32x4*>(tiled + i * 16) = *reinterpret_cast<const u32x4*>(w + n * K + k);
  }
}

__global__ void fp8_unpack_kernel(const uint8_t* __restrict__ tiled, uint8_t* __restrict__ w, int64_t N,
                                  int64_t K) {
  const int64_t KB = K / 128, pieces = N * K / 16;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pieces;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int l = (int)(i & 63), h = (int)((i >> 6) & 1);
    const int64_t tile = i >> 7, kb = tile % KB, nt = tile / KB;
    const int64_t n = nt * 16 + (l & 15), k = kb * 128 + 32 * (l >> 4) + 16 * h;
    *reinterpret_cast<u32x4*>(w + n * K + k) = *reinterpret_cast<const u32x4*>(tiled + i * 16);
  }
}

// ------------------------------------------------------ grouped GEMM --
enum { F8_STORE = 0, F8_ROWS = 1, F8_SILU_Q = 2 };

struct Fp8GP {
  const uint8_t* a;            // activations e4m3fn [*, K]
  int64_t lda;
  const float* sa;             // their scales [*, K/128]
  int64_t ldsa;
  const int32_t* rows;         // per tile 64 row ids (-1 = padding); null = dense rows
  int row_div;                 // activation row = row id / row_div
  const int32_t* tile_expert;  // null = one weight
  const int32_t* meta;         // meta[0] = valid tiles; null = all
  int tile_div;                // kernel tiles per schedule tile (schedule rows / BM)
  const uint8_t* w0;           // tiled weights (gate for F8_SILU_Q)
  const float* sw0;            // block scales [N/128, K/128]
  const uint8_t* w1;           // up weights for F8_SILU_Q
  const float* sw1;
  int64_t w_es, sw_es;         // per-expert strides (bytes, floats)
  void* y;                     // F8_STORE: [M, N] y_dtype; F8_ROWS: float [row id, N]
  int64_t ldy;
  int y_dtype;
  uint8_t* qy;                 // F8_SILU_Q: e4m3fn [row id, N] and scales [row id, N/128]
  float* sy;
  int64_t ldqy, ldsy;
  int M, N, K, KB;
};

constexpr int F8_BM_SMALL = 64;   // rows per tile (decode-sized groups)
constexpr int F8_BM_LARGE = 128;  // rows per tile when experts receive many tokens
constexpr int F8_BN = 128;        // output channels per workgroup (one scale block)
constexpr int F8_ALD = 128 + 16;  // LDS row stride of the A tile (bytes)

__device__ __forceinline__ f32x4 mfma_f8(const i32x8& a, const i32x8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// Workgroup = 8 waves on one BM-row tile x 128 output channels (blockIdx.x =
// channel block, blockIdx.y = tile).  Wave w owns channels [16w, 16w+16)
// (one 16-channel MFMA column; F8_SILU_Q: the same channels of gate and
// up).  Per 128-wide K block: the A tile (BM x 128 bytes) and its row scales
// go through LDS (double-buffered), the wave's weight tiles go straight to
// registers; BM/16 (or 2*BM/16) MFMAs per wave.  Each tile streams its
// expert's whole weight, so the tile height is chosen to hold all of an
// expert's tokens whenever that is affordable (128 for prefill).
constexpr int F8_WAVES = 8;

template <int EPI, int BM>
__global__ __launch_bounds__(512) void fp8_gemm_kernel(const Fp8GP p) {
  constexpr int NQ = EPI == F8_SILU_Q ? 2 : 1;  // weight matrices
  constexpr int NC = NQ;                        // 16-channel B tiles per wave
  constexpr int RT = BM / 16;                   // 16-row MFMA tiles
  constexpr int AP = BM * 8 / (64 * F8_WAVES);  // 16-byte A pieces per thread
  __shared__ __align__(16) uint8_t As[2][BM * F8_ALD];
  __shared__ __align__(16) float Ss[2][BM];
  __shared__ int Rid[BM];
  __shared__ float Red[F8_WAVES][BM];
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
  // a tile of padding only (the tail of an expert's last schedule tile)
  if (!__syncthreads_or(tid < BM && Rid[tid] >= 0)) return;

  // A staging: BM rows x 8 pieces of 16 bytes, AP pieces per thread
  // (piece i = tid + 512*j: row = i / 8, part = i % 8)
  const uint8_t* asrc[AP];
  bool aval[AP];
#pragma unroll
  for (int j = 0; j < AP; ++j) {
    const int i = tid + 64 * F8_WAVES * j, row = i >> 3, part = i & 7;
    aval[j] = Rid[row] >= 0;
    asrc[j] = p.a + (int64_t)(aval[j] ? Rid[row] / p.row_div : 0) * p.lda + 16 * part;
  }
  const float* ssrc = nullptr;
  bool sval = false;
  if (tid < BM) {
    const int rid = Rid[tid];
    sval = rid >= 0;
    ssrc = p.sa + (int64_t)(sval ? rid / p.row_div : 0) * p.ldsa;
  }
  // A for a K block: AP 16-byte pieces per thread (+ one row scale for
  // threads < BM), held in registers until written to LDS
  struct AStage {
    u32x4 v[AP];
    float s;
  };
  auto load_a = [&](AStage& st, int kb) {
#pragma unroll
    for (int j = 0; j < AP; ++j) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(asrc[j] + (int64_t)kb * 128);
      st.v[j] = aval[j] ? v : u32x4{0u, 0u, 0u, 0u};
    }
    if (tid < BM) st.s = sval ? ssrc[kb] : 0.f;
  };
  auto store_a = [&](const AStage& st, int buf) {
#pragma unroll
    for (int j = 0; j < AP; ++j) {
      const int i = tid + 64 * F8_WAVES * j, row = i >> 3, part = i & 7;
      *reinterpret_cast<u32x4*>(&As[buf][row * F8_ALD + 16 * part]) = st.v[j];
    }
    if (tid < BM) Ss[buf][tid] = st.s;
  };
  // weight tile of this wave: channel tile nt = nb*8 + wave, per matrix
  const uint8_t* wsrc[NC];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
    wsrc[q] = (q == 0 ? p.w0 : p.w1) + (int64_t)ex * p.w_es + ((int64_t)(nb * 8 + wave) * p.KB) * 2048 + lane * 16;
  const float* swb[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) swb[q] = (q == 0 ? p.sw0 : p.sw1) + (int64_t)ex * p.sw_es + (int64_t)nb * p.KB;

  auto load_b = [&](i32x8 (&b)[NC], int kb) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const uint8_t* src = wsrc[c] + (int64_t)kb * 2048;
      const u32x4 lo = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
      const u32x4 hi = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + 1024));
      b[c] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
  };

  f32x4 acc[RT][NC];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[rt][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int r = lane & 15, kq = lane >> 4;
  auto compute = [&](int buf, const i32x8 (&b)[NC], int kb) {
    float sw[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) sw[q] = swb[q][kb];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const uint8_t* ap = &As[buf][(rt * 16 + r) * F8_ALD + 32 * kq];
      const u32x4 lo = *reinterpret_cast<const u32x4*>(ap);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(ap + 16);
      const i32x8 a = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      const f32x4 sr = *reinterpret_cast<const f32x4*>(&Ss[buf][rt * 16 + 4 * kq]);
      f32x4 t[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) t[c] = mfma_f8(a, b[c], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float s = sw[c];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[rt][c][i] = fmaf(sr[i] * s, t[c][i], acc[rt][c][i]);
      }
      // keep one row tile's products live at a time (the scheduler would
      // otherwise hoist every MFMA of the block and run out of registers)
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // software pipeline: step kb computes block kb from LDS buffer kb & 1 and
  // a weight register slot, then writes A(kb+1) to LDS; the loads of block
  // kb+DEPTH (A first, then weights) are issued at its start.  Waits retire
  // loads in issue order, so writing A(kb+1) only waits for loads issued up
  // to A(kb+1) itself and the later weights stay in flight.  DEPTH is 2, or
  // 1 where the registers of a third stage would cost a workgroup per CU
  // (measured: two resident workgroups hide each other's barrier stalls
  // better than a deeper single-workgroup pipeline).
  constexpr int DEPTH = (EPI == F8_SILU_Q && BM == F8_BM_LARGE) || EPI == F8_ROWS ? 1 : 2;
  if constexpr (DEPTH == 2) {
    AStage as0, as1, as2;
    i32x8 b0[NC], b1[NC], b2[NC];
    auto step = [&](int kb, AStage& a_next, AStage& a_far, const i32x8 (&bc)[NC], i32x8 (&bfar)[NC]) {
      if (kb + 2 < p.KB) {
        load_a(a_far, kb + 2);
        load_b(bfar, kb + 2);
      }
      compute(kb & 1, bc, kb);
      if (kb + 1 < p.KB) store_a(a_next, (kb + 1) & 1);
      __syncthreads();
    };
    load_a(as0, 0);
    load_b(b0, 0);
    if (p.KB > 1) {
      load_a(as1, 1);
      load_b(b1, 1);
    }
    store_a(as0, 0);
    __syncthreads();
    for (int kb = 0; kb < p.KB; kb += 3) {
      step(kb, as1, as2, b0, b2);
      if (kb + 1 >= p.KB) break;
      step(kb + 1, as2, as0, b1, b0);
      if (kb + 2 >= p.KB) break;
      step(kb + 2, as0, as1, b2, b1);
    }
  } else {
    AStage as0, as1;
    i32x8 b0[NC], b1[NC];
    load_a(as0, 0);
    load_b(b0, 0);
    store_a(as0, 0);
    __syncthreads();
    for (int kb = 0; kb < p.KB; kb += 2) {
      if (kb + 1 < p.KB) {
        load_a(as1, kb + 1);
        load_b(b1, kb + 1);
      }
      compute(0, b0, kb);
      if (kb + 1 < p.KB) store_a(as1, 1);
      __syncthreads();
      if (kb + 1 >= p.KB) break;
      if (kb + 2 < p.KB) {
        load_a(as0, kb + 2);
        load_b(b0, kb + 2);
      }
      compute(1, b1, kb + 1);
      if (kb + 2 < p.KB) store_a(as0, 0);
      __syncthreads();
    }
  }

  // epilogue: lane holds rows rt*16 + 4*kq + i, channel c*16 + r of its wave
  if constexpr (EPI == F8_SILU_Q) {
    float h[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float g = acc[rt][0][i], u = acc[rt][1][i];
        // silu(g) * u in float64 stored float32 (kernels.py:219-231), then
        // rounded to bf16: the intermediate is held in bf16
        const double gd = (double)g;
        const float hv = (float)((gd / (1.0 + exp(-gd))) * (double)u);
        const float hb = bf16_bits_to_f32(f32_to_bf16_bits(hv));
        h[rt][i] = hb;
        float m = fabsf(hb);
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        if (r == 0) Red[wave][rt * 16 + 4 * kq + i] = m;
      }
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = rt * 16 + 4 * kq + i;
        const int rid = Rid[row];
        if (rid < 0) continue;
        float amax = Red[0][row];
#pragma unroll
        for (int w = 1; w < F8_WAVES; ++w) amax = fmaxf(amax, Red[w][row]);
        const float sc = fmaxf(amax, kAmaxFloor) / kFp8Max;
        const int64_t col = (int64_t)nb * F8_BN + 16 * wave + r;
        p.qy[(int64_t)rid * p.ldqy + col] = (uint8_t)f32_to_fp8_rne(h[rt][i] / sc);
        if (wave == 0 && r == 0) p.sy[(int64_t)rid * p.ldsy + nb] = sc;
      }
  } else {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rid = Rid[rt * 16 + 4 * kq + i];
        if (rid < 0) continue;
        const int64_t col = (int64_t)nb * F8_BN + 16 * wave + r;
        const int64_t o = (int64_t)rid * p.ldy + col;
        const float v = acc[rt][0][i];
        if (EPI == F8_ROWS || p.y_dtype == CCQ_F32)
          reinterpret_cast<float*>(p.y)[o] = v;
        else if (p.y_dtype == CCQ_BF16)
          reinterpret_cast<uint16_t*>(p.y)[o] = (uint16_t)f32_to_bf16_bits(v);
        else
          reinterpret_cast<uint16_t*>(p.y)[o] = (uint16_t)f32_to_f16_bits(v);
      }
  }
}

static int grid_of(int64_t n, int block) {
  const int64_t g = cdiv(n, block);
  return (int)(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

int launch_act_quant(const void* x, int x_dtype, int64_t ldx, int64_t rows, int64_t K, uint8_t* q, int64_t ldq,
                     float* s, int64_t lds_, hipStream_t st) {
  const int64_t KB = K / 128;
  const dim3 grid(grid_of(rows * KB * 16, 256));
  if (x_dtype == CCQ_BF16)
    hipLaunchKernelGGL(fp8_act_quant_kernel<CCQ_BF16>, grid, dim3(256), 0, st, x, ldx, q, ldq, s, lds_, rows, KB);
  else if (x_dtype == CCQ_F16)
    hipLaunchKernelGGL(fp8_act_quant_kernel<CCQ_F16>, grid, dim3(256), 0, st, x, ldx, q, ldq, s, lds_, rows, KB);
  else
    hipLaunchKernelGGL(fp8_act_quant_kernel<CCQ_F32>, grid, dim3(256), 0, st, x, ldx, q, ldq, s, lds_, rows, KB);
  return launch_status("fp8 act quant");
}

// bm: rows per schedule tile; kernel_bm: rows per kernel tile (a divisor)
template <int EPI>
static int launch_fp8_gemm(Fp8GP p, int bm, int kernel_bm, int64_t tiles, hipStream_t st) {
  p.tile_div = bm / kernel_bm;
  const dim3 grid((unsigned)(p.N / F8_BN), (unsigned)(tiles * p.tile_div)), block(64 * F8_WAVES);
  if (kernel_bm == F8_BM_LARGE)
    hipLaunchKernelGGL((fp8_gemm_kernel<EPI, F8_BM_LARGE>), grid, block, 0, st, p);
  else
    hipLaunchKernelGGL((fp8_gemm_kernel<EPI, F8_BM_SMALL>), grid, block, 0, st, p);
  return launch_status("fp8 gemm");
}

// Tile height of a grouped call: 128 rows once the average expert receives
// at least 32 tokens (each tile re-streams its expert's weights, so a tile
// should hold all of them), 64 below that.
static int fp8_tile_rows(int64_t assignments, int64_t experts) {
  return assignments >= 32 * experts ? F8_BM_LARGE : F8_BM_SMALL;
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
  CCQ_REQUIRE(N % 16 == 0 && K % 128 == 0, "ccq_fp8_block_repack: need N %% 16 == 0 and K %% 128 == 0");
  if (N == 0 || K == 0) return 0;
  CCQ_REQUIRE(w && tiled, "ccq_fp8_block_repack: null pointer");
  CCQ_REQUIRE(w != tiled, "ccq_fp8_block_repack: in-place is not supported");
  CCQ_REQUIRE(aligned(w, 16) && aligned(tiled, 16), "ccq_fp8_block_repack: pointers must be 16-byte aligned");
  hipLaunchKernelGGL(fp8_repack_kernel, dim3(grid_of(N * K / 16, 256)), dim3(256), 0, as_stream(stream), w, tiled,
                     N, K);
  return launch_status("ccq_fp8_block_repack");
}

extern "C" int ccq_fp8_block_unpack(const uint8_t* tiled, uint8_t* w, int64_t N, int64_t K, void* stream) {
  CCQ_REQUIRE(N >= 0 && K >= 0, "ccq_fp8_block_unpack: negative shape");
  CCQ_REQUIRE(N % 16 == 0 && K % 128 == 0, "ccq_fp8_block_unpack: need N %% 16 == 0 and K %% 128 == 0");
  if (N == 0 || K == 0) return 0;
  CCQ_REQUIRE(w && tiled, "ccq_fp8_block_unpack: null pointer");
  CCQ_REQUIRE(w != tiled, "ccq_fp8_block_unpack: in-place is not supported");
  CCQ_REQUIRE(aligned(w, 16) && aligned(tiled, 16), "ccq_fp8_block_unpack: pointers must be 16-byte aligned");
  hipLaunchKernelGGL(fp8_unpack_kernel, dim3(grid_of(N * K / 16, 256)), dim3(256), 0, as_stream(stream), tiled, w,
                     N, K);
  return launch_status("ccq_fp8_block_unpack");
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
  CCQ_REQUIRE(cdiv(M, F8_BM_SMALL) <= 65535 && N / F8_BN <= 65535, "ccq_fp8_block_linear: M or N too large");
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
  const int bm = M >= F8_BM_LARGE ? F8_BM_LARGE : F8_BM_SMALL;
  return launch_fp8_gemm<F8_STORE>(p, bm, bm, cdiv(M, bm), st);
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
  CCQ_REQUIRE(ex->hidden / F8_BN <= 65535 && ex->inter / F8_BN <= 65535, "%s: hidden/inter too large", name);
  CCQ_REQUIRE(ex->w_gate && ex->s_gate && ex->w_up && ex->s_up && ex->w_down && ex->s_down,
              "%s: null weight pointer", name);
  CCQ_REQUIRE(aligned(ex->w_gate, 16) && aligned(ex->w_up, 16) && aligned(ex->w_down, 16),
              "%s: tiled weights must be 16-byte aligned", name);
  return 0;
}

struct F8MoeLayout {
  int64_t n, max_tiles;
  int bm;
  size_t off_sorted, off_te, off_meta, off_counts, off_qx, off_sx, off_qh, off_sh, off_rows, total;
};

F8MoeLayout f8_moe_layout(int64_t T, int64_t k, const ccq_fp8_experts* ex) {
  F8MoeLayout L;
  const int64_t H = ex->hidden, I = ex->inter;
  L.n = T * k;
  L.bm = fp8_tile_rows(L.n, ex->num_experts);
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
  L.off_sh = o;
  o += a256((size_t)L.n * (I / 128) * 4);
  L.off_rows = o;
  o += a256((size_t)L.n * H * 4);
  L.total = o;
  return L;
}

}  // namespace

extern "C" size_t ccq_moe_fp8_workspace_size(int64_t T, int64_t k, const ccq_fp8_experts* ex) {
  if (T <= 0 || k <= 0 || check_fp8_experts(ex, "ccq_moe_fp8_workspace_size") != 0) return 0;
  return f8_moe_layout(T, k, ex).total;
}

extern "C" int ccq_moe_fp8_ffn(const void* x, int x_dtype, const int64_t* ids, const float* weights, void* y,
                               int y_dtype, int64_t T, int64_t k, const ccq_fp8_experts* ex, void* workspace,
                               size_t workspace_bytes, void* stream) {
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
  CCQ_REQUIRE(L.max_tiles * 2 <= 65535, "ccq_moe_fp8_ffn: too many tiles");
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
  float* sh = (float*)(ws + L.off_sh);
  float* rows = (float*)(ws + L.off_rows);

  rc = launch_align(ids, L.n, ex->num_experts, L.bm, sorted, te, meta, counts, st);
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
  g.sy = sh;
  g.ldqy = I;
  g.ldsy = I / 128;
  g.N = (int)I;
  g.K = (int)H;
  g.KB = (int)(H / 128);
  rc = launch_fp8_gemm<F8_SILU_Q>(g, L.bm, L.bm, L.max_tiles, st);
  if (rc) return rc;

  Fp8GP d = {};
  d.a = qh;
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
  d.y_dtype = CCQ_F32;
  d.N = (int)H;
  d.K = (int)I;
  d.KB = (int)(I / 128);
  // down runs 64-row tiles (two resident workgroups per CU; see DEPTH)
  rc = launch_fp8_gemm<F8_ROWS>(d, L.bm, F8_BM_SMALL, L.max_tiles, st);
  if (rc) return rc;
  return launch_combine(rows, CCQ_F32, weights, ids, ex->num_experts, y, y_dtype, T, k, H, st);
}
