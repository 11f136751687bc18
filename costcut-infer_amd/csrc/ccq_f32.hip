// Float32 GEMM on the fp32 matrix cores (v_mfma_f32_16x16x4_f32) for the
// reference's float32 products that run on already-float32 operands:
//   * the router x @ gate_w.T (experts/pipeline.py:145): w given [N, K];
//   * expert_ffn's x @ W_gate, x @ W_up, h @ W_down on dequantized float32
//     weights (blocks/moe.py:122-141): w given [K, N];
//   * the same per expert over the expert-sorted schedule, for readers that
//     hand over float32 slots (experts/pipeline.py:155-179), with the
//     experts' weights found through device tables of pointers.
// The products are float32 (no rounding of the operands), accumulated in
// float32 by the matrix core in an order of its own; the SiLU product of
// the gate/up stage is formed in float64 and rounded once, as the
// reference's silu_mul_fused (quant/kernels.py:219-231).
//
// Tiling: a workgroup of 4 waves owns a 64 x 64 block of the output; K runs
// in slabs of 16, double-buffered in LDS with one barrier per slab, the
// next two slabs' loads in flight in registers while the current one is
// multiplied.  The
// A slab is stored k-major ([k][row]) and the B slab [k][col], so the 16
// lanes that read one MFMA operand column touch 16 consecutive words.  Wave
// (wr, wc) computes rows 32 wr .. +31 x columns 32 wc .. +31 as 2 x 2 MFMA
// tiles.  Loads are 16-byte (float4) when the shapes and pointers allow,
// else per element; every element past M, N or K reads as zero.  The
// grouped form's 16-byte loads of B need every table pointer 16-byte
// aligned (the caller guarantees it).
#include "ccq_common.h"

namespace ccq {

constexpr int FG_BM = 64, FG_BN = 64, FG_BK = 16, FG_THREADS = 256;
// LDS row stride in floats: an MFMA operand read takes 16 consecutive words
// from each of 4 slab rows; 16 words of padding put the 4 rows' words in
// distinct banks (unpadded, all 4 rows map to the same 16 banks)
constexpr int FG_RS = FG_BM + 16;

struct F32GP {
  const float* a;               // A [rows, K] (row stride lda)
  int64_t lda;
  const int32_t* rows;          // grouped: expert-sorted assignment ids per tile row (-1 padding), else null
  int row_div;                  // grouped: A row of assignment r = r / row_div
  const int32_t* tile_expert;   // grouped: expert of each 64-row tile
  const int32_t* meta;          // grouped: meta[0] = tiles
  const float* b0;              // dense B (gate or the only one)
  const float* b1;              // dense B of the second product (DUAL)
  const float* const* tab0;     // grouped: per-expert B pointers (null entry: the expert's rows are zero)
  const float* const* tab1;
  int64_t ldb;
  float* c;                     // output rows (dense: row m; grouped: row = assignment id)
  int64_t ldc;
  int64_t M, N, K;              // M: rows of a dense product
  int64_t kchunk;               // K per split (gridDim.z splits); partial sums to c + split * M * ldc
};

// 4 consecutive floats at p, of which `avail` (may be <= 0) are in bounds
template <bool VEC>
__device__ __forceinline__ float4 ld4(const float* p, int64_t avail) {
  if constexpr (VEC) {
    return avail >= 4 ? *reinterpret_cast<const float4*>(p) : make_float4(0.f, 0.f, 0.f, 0.f);
  } else {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (avail > 0) v.x = p[0];
    if (avail > 1) v.y = p[1];
    if (avail > 2) v.z = p[2];
    if (avail > 3) v.w = p[3];
    return v;
  }
}

// BT: B given as [N, K] (y = A @ B^T); else [K, N].  DUAL: two B operands and
// the SiLU product epilogue.  GROUPED: rows gathered through the schedule.
template <bool BT, bool DUAL, bool GROUPED, bool VEC>
__global__ __launch_bounds__(FG_THREADS) void f32_gemm_kernel(const F32GP p) {
  constexpr int NB = DUAL ? 2 : 1;
  static_assert(FG_BM == FG_BN, "one LDS row stride for both slabs");
  __shared__ __align__(16) float As[2][FG_BK][FG_RS];
  __shared__ __align__(16) float Bs[2][NB][FG_BK][FG_RS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t N = p.N;
  // split z of gridDim.z: k in [kbeg, kbeg + K), written to its own partial slice
  const int64_t kbeg = (int64_t)blockIdx.z * p.kchunk;
  const int64_t K = imin64(p.kchunk, p.K - kbeg);
  float* const cout = p.c + (int64_t)blockIdx.z * p.M * p.ldc;
  const int64_t n0 = (int64_t)blockIdx.x * FG_BN;
  const float* b0 = p.b0;
  const float* b1 = p.b1;
  const int32_t* trow = nullptr;
  int64_t m0 = 0;
  if constexpr (GROUPED) {
    const int tile = blockIdx.y;
    if (tile >= p.meta[0]) return;  // uniform
    const int e = p.tile_expert[tile];
    b0 = p.tab0[e];
    if constexpr (DUAL) b1 = p.tab1[e];
    trow = p.rows + (int64_t)tile * FG_BM;
    if (b0 == nullptr || (DUAL && b1 == nullptr)) {  // an expert without weights: its rows are zero
      for (int i = tid; i < FG_BM * FG_BN; i += FG_THREADS) {
        const int r = i / FG_BN;
        const int64_t n = n0 + i % FG_BN;
        const int a = trow[r];
        if (a >= 0 && n < N) p.c[(int64_t)a * p.ldc + n] = 0.f;
      }
      return;
    }
  } else {
    m0 = (int64_t)blockIdx.y * FG_BM;
  }

  // A: thread loads row tid % 64, k 4 (tid / 64) .. +3 of the slab
  const int am = tid & 63, ak = 4 * (tid >> 6);
  const float* arow = nullptr;
  bool a_ok;
  if constexpr (GROUPED) {
    const int a = trow[am];
    a_ok = a >= 0;
    arow = p.a + (int64_t)(a_ok ? a / p.row_div : 0) * p.lda + kbeg;
  } else {
    a_ok = m0 + am < p.M;
    arow = p.a + (a_ok ? m0 + am : 0) * p.lda + kbeg;
  }
  b0 += BT ? kbeg : kbeg * p.ldb;
  if constexpr (DUAL) b1 += BT ? kbeg : kbeg * p.ldb;
  // B [K, N]: thread loads k tid / 16, columns 4 (tid % 16) .. +3;
  // B [N, K]: thread loads column tid % 64, k 4 (tid / 64) .. +3
  const int bk = BT ? 4 * (tid >> 6) : (tid >> 4);
  const int bn = BT ? (tid & 63) : 4 * (tid & 15);

  float4 ra, rb0, rb1;
  auto load = [&](int64_t k0) {
    ra = a_ok ? ld4<VEC>(arow + k0 + ak, K - (k0 + ak)) : make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (BT) {
      const bool ok = n0 + bn < N;
      const int64_t off = (ok ? n0 + bn : 0) * p.ldb + k0 + bk;
      rb0 = ok ? ld4<VEC>(b0 + off, K - (k0 + bk)) : make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (DUAL) rb1 = ok ? ld4<VEC>(b1 + off, K - (k0 + bk)) : make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
      const bool ok = k0 + bk < K;
      const int64_t off = (ok ? k0 + bk : 0) * p.ldb + n0 + bn;
      rb0 = ok ? ld4<VEC>(b0 + off, N - (n0 + bn)) : make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (DUAL) rb1 = ok ? ld4<VEC>(b1 + off, N - (n0 + bn)) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto store = [&](int buf) {
    As[buf][ak + 0][am] = ra.x;
    As[buf][ak + 1][am] = ra.y;
    As[buf][ak + 2][am] = ra.z;
    As[buf][ak + 3][am] = ra.w;
    if constexpr (BT) {
      Bs[buf][0][bk + 0][bn] = rb0.x;
      Bs[buf][0][bk + 1][bn] = rb0.y;
      Bs[buf][0][bk + 2][bn] = rb0.z;
      Bs[buf][0][bk + 3][bn] = rb0.w;
      if constexpr (DUAL) {
        Bs[buf][NB - 1][bk + 0][bn] = rb1.x;
        Bs[buf][NB - 1][bk + 1][bn] = rb1.y;
        Bs[buf][NB - 1][bk + 2][bn] = rb1.z;
        Bs[buf][NB - 1][bk + 3][bn] = rb1.w;
      }
    } else {
      *reinterpret_cast<float4*>(&Bs[buf][0][bk][bn]) = rb0;
      if constexpr (DUAL) *reinterpret_cast<float4*>(&Bs[buf][NB - 1][bk][bn]) = rb1;
    }
  };

  const int wr = wave >> 1, wc = wave & 1, c16 = lane & 15, q = lane >> 4;
  f32x4 acc[NB][2][2];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[b][i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto mma = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < FG_BK; kk += 4) {
      float av[2], bv[NB][2];
#pragma unroll
      for (int i = 0; i < 2; ++i) av[i] = As[buf][kk + q][32 * wr + 16 * i + c16];
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int j = 0; j < 2; ++j) bv[b][j] = Bs[buf][b][kk + q][32 * wc + 16 * j + c16];
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[b][i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[b][j], acc[b][i][j], 0, 0, 0);
    }
  };

  // slab s + 1 is in LDS buffer (s + 1) & 1 before slab s's products end,
  // and slab s + 2's loads are in flight meanwhile (two register sets, the
  // loop unrolled by two so that each set has fixed registers)
  const int64_t nslab = cdiv(K, FG_BK);
  load(0);
  store(0);
  float4 xa = ra, xb0 = rb0, xb1 = rb1;  // register set of odd slabs
  if (nslab > 1) {
    load(FG_BK);
    xa = ra, xb0 = rb0, xb1 = rb1;
  }
  __syncthreads();
  for (int64_t s = 0; s < nslab; s += 2) {
    // even slab s in LDS 0, slab s + 1 in (xa, xb0, xb1)
    if (s + 2 < nslab) load((s + 2) * FG_BK);
    mma(0);
    if (s + 1 < nslab) {
      float4 ta = ra, tb0 = rb0, tb1 = rb1;
      ra = xa, rb0 = xb0, rb1 = xb1;
      store(1);
      ra = ta, rb0 = tb0, rb1 = tb1;
    }
    __syncthreads();
    if (s + 1 >= nslab) break;
    // odd slab s + 1 in LDS 1, slab s + 2 in (ra, rb0, rb1)
    if (s + 3 < nslab) {
      const float4 ta = ra, tb0 = rb0, tb1 = rb1;
      load((s + 3) * FG_BK);
      xa = ra, xb0 = rb0, xb1 = rb1;
      ra = ta, rb0 = tb0, rb1 = tb1;
    }
    mma(1);
    if (s + 2 < nslab) store(0);
    __syncthreads();
  }

  // lane (c16, q) of tile (i, j): column 32 wc + 16 j + c16, rows 32 wr + 16 i + 4 q + t
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t n = n0 + 32 * wc + 16 * j + c16;
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int r = 32 * wr + 16 * i + 4 * q + t;
        int64_t orow;
        if constexpr (GROUPED) {
          const int a = trow[r];
          if (a < 0) continue;
          orow = a;
        } else {
          orow = m0 + r;
          if (orow >= p.M) continue;
        }
        float v;
        if constexpr (DUAL) {
          const double g = acc[0][i][j][t], u = acc[NB - 1][i][j][t];
          v = (float)(g / (1.0 + exp(-g)) * u);
        } else {
          v = acc[0][i][j][t];
        }
        cout[orow * p.ldc + n] = v;
      }
  }
}

// y = the sum of `splits` partial products in split order (deterministic)
__global__ __launch_bounds__(256) void f32_splitk_sum_kernel(const float* __restrict__ part, float* __restrict__ y,
                                                             int64_t n, int splits) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    float v = part[i];
    for (int s = 1; s < splits; ++s) v += part[(int64_t)s * n + i];
    y[i] = v;
  }
}

template <bool BT, bool DUAL, bool GROUPED>
static int f32_launch(F32GP p, int64_t tiles_y, bool vec, hipStream_t st, const char* name, int splits = 1) {
  if (splits == 1) p.kchunk = p.K;
  const dim3 grid((unsigned)cdiv(p.N, FG_BN), (unsigned)tiles_y, (unsigned)splits);
  if (vec)
    launch((f32_gemm_kernel<BT, DUAL, GROUPED, true>), grid, dim3(FG_THREADS), 0, st, p);
  else
    launch((f32_gemm_kernel<BT, DUAL, GROUPED, false>), grid, dim3(FG_THREADS), 0, st, p);
  return launch_status(name);
}

// float4 loads are exact (never straddle the bounds) when K (and N for a
// [K, N] B) and the row strides are multiples of 4 and the bases are
// 16-byte aligned
static bool f32_vec_ok(const float* a, int64_t lda, const void* b, int64_t ldb, bool bt, int64_t K, int64_t N) {
  return aligned(a, 16) && (b == nullptr || aligned(b, 16)) && lda % 4 == 0 && ldb % 4 == 0 && K % 4 == 0 &&
         (bt || N % 4 == 0);
}


// y [M, N] = x [M, K] @ w^T for w [N, K] and few rows (the router at decode
// batch sizes): the tiled kernel would be one workgroup walking K.  Here a
// workgroup is 4 waves x RT weight rows (output columns); lane l streams
// floats 4 l + 256 i of each of its rows in 16-byte pieces, all of a row's
// pieces in flight at once for K <= 2048; BB rows of x per pass are staged
// in LDS (zeros past M); the per-lane products of the RT x BB outputs are
// summed over the wave by halving exchanges, in a fixed order.  Requires
// K % 4 == 0 and 16-byte aligned x, w.
constexpr int FS_RT = 2;
constexpr int FS_LDS = 64 * 1024;

template <int V>
__device__ __forceinline__ float fs_wave_sum(float (&v)[V], int lane) {
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
  return t;  // lane l: the sum of value l % V
}

template <int BB>
__global__ __launch_bounds__(256) void f32_skinny_nt_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                            float* __restrict__ y, int64_t M, int64_t K, int64_t N) {
  extern __shared__ __align__(16) float xs[];  // [BB][K]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t m0 = (int64_t)blockIdx.y * BB;
  const int nb = (int)imin64(BB, M - m0);
  const int64_t q4 = K / 4, nq = BB * q4;
  for (int64_t i0 = 0; i0 < nq; i0 += 8 * 256) {  // 8 loads in flight per thread
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t i = i0 + 256 * u + tid, b = i / q4;
      v[u] = i < nq && b < nb ? *reinterpret_cast<const float4*>(x + (m0 + b) * K + 4 * (i - b * q4))
                              : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t i = i0 + 256 * u + tid;
      if (i < nq) *reinterpret_cast<float4*>(&xs[4 * i]) = v[u];
    }
  }
  __syncthreads();
  const int64_t n0 = ((int64_t)blockIdx.x * 4 + wave) * FS_RT;
  if (n0 >= N) return;
  const float* wr[FS_RT];
#pragma unroll
  for (int r = 0; r < FS_RT; ++r) wr[r] = w + imin64(n0 + r, N - 1) * K;  // past N: row N-1, not stored
  float acc[FS_RT][BB];
#pragma unroll
  for (int r = 0; r < FS_RT; ++r)
#pragma unroll
    for (int b = 0; b < BB; ++b) acc[r][b] = 0.f;
  constexpr int U = 8;  // pieces per row in flight
  for (int64_t k0 = 4 * lane; k0 < K; k0 += 256 * U) {
    float4 wv[U][FS_RT];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < FS_RT; ++r)
        wv[u][r] = k0 + 256 * u < K
                       ? __builtin_bit_cast(float4, __builtin_nontemporal_load(
                                                        reinterpret_cast<const f32x4*>(wr[r] + k0 + 256 * u)))
                       : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (k0 + 256 * u >= K) break;
#pragma unroll
      for (int b = 0; b < BB; ++b) {
        const float4 xv = *reinterpret_cast<const float4*>(&xs[b * K + k0 + 256 * u]);
#pragma unroll
        for (int r = 0; r < FS_RT; ++r) {
          acc[r][b] = fmaf(xv.x, wv[u][r].x, acc[r][b]);
          acc[r][b] = fmaf(xv.y, wv[u][r].y, acc[r][b]);
          acc[r][b] = fmaf(xv.z, wv[u][r].z, acc[r][b]);
          acc[r][b] = fmaf(xv.w, wv[u][r].w, acc[r][b]);
        }
      }
    }
  }
  float flat[FS_RT * BB];
#pragma unroll
  for (int r = 0; r < FS_RT; ++r)
#pragma unroll
    for (int b = 0; b < BB; ++b) flat[r * BB + b] = acc[r][b];
  const float v = fs_wave_sum<FS_RT * BB>(flat, lane);
  if (lane < FS_RT * BB) {
    const int r = lane / BB, b = lane % BB;
    if (n0 + r < N && b < nb) y[(m0 + b) * N + n0 + r] = v;
  }
}

// rows per pass of the skinny kernel (0: not taken): the fewest passes
// whose x rows fit the LDS; every pass re-reads w, so at most 4 passes
static int f32_skinny_bb(int64_t M, int64_t K) {
  int bb = 1;
  while (bb < 16 && bb < M && (int64_t)(2 * bb) * K * 4 <= FS_LDS) bb *= 2;
  if ((int64_t)bb * K * 4 > FS_LDS) return 0;
  return cdiv(M, bb) <= 4 ? bb : 0;
}

static int f32_skinny_launch(int bb, const float* x, const float* w, float* y, int64_t M, int64_t K, int64_t N,
                             hipStream_t st) {
  const dim3 grid((unsigned)cdiv(N, 4 * FS_RT), (unsigned)cdiv(M, bb));
  const size_t lds = (size_t)bb * K * 4;
  switch (bb) {
    case 1: launch((f32_skinny_nt_kernel<1>), grid, dim3(256), lds, st, x, w, y, M, K, N); break;
    case 2: launch((f32_skinny_nt_kernel<2>), grid, dim3(256), lds, st, x, w, y, M, K, N); break;
    case 4: launch((f32_skinny_nt_kernel<4>), grid, dim3(256), lds, st, x, w, y, M, K, N); break;
    case 8: launch((f32_skinny_nt_kernel<8>), grid, dim3(256), lds, st, x, w, y, M, K, N); break;
    default: launch((f32_skinny_nt_kernel<16>), grid, dim3(256), lds, st, x, w, y, M, K, N); break;
  }
  return launch_status("ccq_f32_gemm (skinny)");
}

namespace {

struct F32MoeLayout {
  int64_t n, max_tiles;
  size_t off_sorted, off_tile_expert, off_meta, off_counts, off_inter, off_rows, off_align, total;
};

size_t a256f(size_t b) { return (b + 255) & ~(size_t)255; }

F32MoeLayout f32_moe_layout(int64_t T, int64_t k, int64_t E, int64_t H, int64_t I) {
  F32MoeLayout L = {};
  L.n = T * k;
  L.max_tiles = ccq_moe_align_max_tiles(L.n, E, FG_BM);
  size_t o = 0;
  L.off_sorted = o;
  o += a256f((size_t)L.max_tiles * FG_BM * 4);
  L.off_tile_expert = o;
  o += a256f((size_t)L.max_tiles * 4);
  L.off_meta = o;
  o += 256;
  L.off_counts = o;
  o += a256f((size_t)E * 4);
  L.off_inter = o;
  o += a256f((size_t)L.n * I * 4);
  L.off_rows = o;
  o += a256f((size_t)L.n * H * 4);
  L.off_align = o;
  o += a256f(align_scratch_bytes(L.n, E));
  L.total = o;
  return L;
}

}  // namespace

}  // namespace ccq

using namespace ccq;

// K splits of the tiled kernel: enough (64 x 64 tile, split) items for two
// per compute unit, each split at least 256 deep (a multiple of the slab)
static int64_t f32_kchunk(int64_t M, int64_t K, int64_t N) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  const int64_t tiles = cdiv(M, FG_BM) * cdiv(N, FG_BN);
  int64_t splits = cdiv(2 * (int64_t)cus, tiles);
  if (splits > K / 256) splits = K / 256;
  if (splits <= 1) return K;
  return cdiv(cdiv(K, splits), FG_BK) * FG_BK;
}

extern "C" size_t ccq_f32_gemm_workspace_size(int64_t M, int64_t K, int64_t N) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  const int64_t kc = f32_kchunk(M, K, N);
  return kc >= K ? 0 : (size_t)cdiv(K, kc) * M * N * 4;
}

extern "C" int ccq_f32_gemm(const float* x, const float* w, float* y, int64_t M, int64_t K, int64_t N, int trans_w,
                            void* workspace, size_t workspace_bytes, void* stream) {
  CCQ_REQUIRE(M >= 0 && K >= 0 && N >= 0, "ccq_f32_gemm: negative shape");
  CCQ_REQUIRE(trans_w == 0 || trans_w == 1, "ccq_f32_gemm: trans_w=%d (0: w [K, N], 1: w [N, K])", trans_w);
  if (M == 0 || N == 0) return 0;
  CCQ_REQUIRE(x && w && y, "ccq_f32_gemm: null pointer");
  CCQ_REQUIRE(cdiv(M, FG_BM) <= 65535, "ccq_f32_gemm: M=%lld too large", (long long)M);
  F32GP p = {};
  p.a = x;
  p.lda = K;
  p.b0 = w;
  p.ldb = trans_w ? K : N;
  p.c = y;
  p.ldc = N;
  p.M = M;
  p.N = N;
  p.K = K;
  const bool vec = f32_vec_ok(x, K, w, p.ldb, trans_w, K, N);
  hipStream_t st = as_stream(stream);
  if (trans_w && vec) {
    const int bb = f32_skinny_bb(M, K);
    if (bb > 0 && cdiv(M, bb) <= 65535) return f32_skinny_launch(bb, x, w, y, M, K, N, st);
  }
  const int64_t kc = f32_kchunk(M, K, N);
  const int64_t splits = cdiv(K, kc);
  const bool split = splits > 1 && workspace != nullptr && workspace_bytes >= (size_t)splits * M * N * 4 &&
                     aligned(workspace, 16) && splits <= 65535;
  if (split) {  // partial products per K range, then their sum in split order
    p.c = (float*)workspace;
    p.kchunk = kc;
  }
  const int sp = split ? (int)splits : 1;
  int rc = trans_w ? f32_launch<true, false, false>(p, cdiv(M, FG_BM), vec, st, "ccq_f32_gemm", sp)
                   : f32_launch<false, false, false>(p, cdiv(M, FG_BM), vec, st, "ccq_f32_gemm", sp);
  if (rc || !split) return rc;
  launch(f32_splitk_sum_kernel, dim3(grid_for(M * N, 256)), dim3(256), 0, st, (const float*)workspace, y, M * N, sp);
  return launch_status("ccq_f32_gemm (split-K sum)");
}

extern "C" size_t ccq_expert_ffn_f32_workspace_size(int64_t rows, int64_t inter) {
  return rows <= 0 || inter <= 0 ? 0 : (size_t)rows * inter * 4;
}

extern "C" int ccq_expert_ffn_f32(const float* x, const float* w_gate, const float* w_up, const float* w_down,
                                  float* y, int64_t rows, int64_t hidden, int64_t inter, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  CCQ_REQUIRE(rows >= 0 && hidden > 0 && inter > 0, "ccq_expert_ffn_f32: bad shape rows=%lld hidden=%lld inter=%lld",
              (long long)rows, (long long)hidden, (long long)inter);
  if (rows == 0) return 0;
  CCQ_REQUIRE(x && w_gate && w_up && w_down && y, "ccq_expert_ffn_f32: null pointer");
  CCQ_REQUIRE(cdiv(rows, FG_BM) <= 65535, "ccq_expert_ffn_f32: rows=%lld too large", (long long)rows);
  CCQ_REQUIRE(workspace && workspace_bytes >= (size_t)rows * inter * 4 && aligned(workspace, 16),
              "ccq_expert_ffn_f32: workspace of %lld bytes (16-byte aligned) needed", (long long)(rows * inter * 4));
  hipStream_t st = as_stream(stream);
  float* h = (float*)workspace;
  F32GP g = {};
  g.a = x;
  g.lda = hidden;
  g.b0 = w_gate;
  g.b1 = w_up;
  g.ldb = inter;
  g.c = h;
  g.ldc = inter;
  g.M = rows;
  g.N = inter;
  g.K = hidden;
  const bool vg = f32_vec_ok(x, hidden, w_gate, inter, false, hidden, inter) && aligned(w_up, 16);
  int rc = f32_launch<false, true, false>(g, cdiv(rows, FG_BM), vg, st, "ccq_expert_ffn_f32 gate/up");
  if (rc) return rc;
  F32GP d = {};
  d.a = h;
  d.lda = inter;
  d.b0 = w_down;
  d.ldb = hidden;
  d.c = y;
  d.ldc = hidden;
  d.M = rows;
  d.N = hidden;
  d.K = inter;
  const bool vd = f32_vec_ok(h, inter, w_down, hidden, false, inter, hidden);
  return f32_launch<false, false, false>(d, cdiv(rows, FG_BM), vd, st, "ccq_expert_ffn_f32 down");
}

extern "C" size_t ccq_moe_f32_workspace_size(int64_t T, int64_t k, int64_t num_experts, int64_t hidden,
                                             int64_t inter) {
  if (T <= 0 || k <= 0 || num_experts <= 0 || hidden <= 0 || inter <= 0) return 0;
  return f32_moe_layout(T, k, num_experts, hidden, inter).total;
}

extern "C" int ccq_moe_f32_ffn(const float* x, const int64_t* ids, const float* weights,
                               const float* const* w_gate, const float* const* w_up, const float* const* w_down,
                               const float* shared, float shared_gate, void* y, int y_dtype, int64_t T, int64_t k,
                               int64_t num_experts, int64_t hidden, int64_t inter, void* workspace,
                               size_t workspace_bytes, void* stream) {
  const int64_t E = num_experts, H = hidden, I = inter;
  CCQ_REQUIRE(T >= 0 && T <= 65535 && k >= 1 && E >= 1 && E <= 1024 && H > 0 && I > 0,
              "ccq_moe_f32_ffn: bad T=%lld k=%lld E=%lld hidden=%lld inter=%lld", (long long)T, (long long)k,
              (long long)E, (long long)H, (long long)I);
  CCQ_REQUIRE(T * k <= 65536, "ccq_moe_f32_ffn: T*k=%lld > 65536", (long long)(T * k));
  CCQ_REQUIRE(y_dtype == CCQ_F32 || y_dtype == CCQ_F16 || y_dtype == CCQ_BF16, "ccq_moe_f32_ffn: bad y_dtype");
  if (T == 0) return 0;
  CCQ_REQUIRE(x && ids && weights && w_gate && w_up && w_down && y, "ccq_moe_f32_ffn: null pointer");
  const F32MoeLayout L = f32_moe_layout(T, k, E, H, I);
  CCQ_REQUIRE(L.max_tiles >= 1 && L.max_tiles <= 65535, "ccq_moe_f32_ffn: too many tiles");
  CCQ_REQUIRE(workspace && workspace_bytes >= L.total && aligned(workspace, 256),
              "ccq_moe_f32_ffn: workspace of %zu bytes (256-byte aligned) needed, %zu given", L.total,
              workspace_bytes);
  hipStream_t st = as_stream(stream);
  char* ws = (char*)workspace;
  int32_t* sorted = (int32_t*)(ws + L.off_sorted);
  int32_t* tile_expert = (int32_t*)(ws + L.off_tile_expert);
  int32_t* meta = (int32_t*)(ws + L.off_meta);
  int32_t* counts = (int32_t*)(ws + L.off_counts);
  float* inter_rows = (float*)(ws + L.off_inter);
  float* rows = (float*)(ws + L.off_rows);
  int rc = launch_align(ids, L.n, E, FG_BM, sorted, tile_expert, meta, counts, st, ws + L.off_align,
                        L.total - L.off_align);
  if (rc) return rc;
  // expert weights may sit anywhere: 16-byte loads only when every row
  // stride allows them (the table's pointers themselves come from
  // allocators that align to 256 bytes; checked on the host by the caller)
  F32GP g = {};
  g.a = x;
  g.lda = H;
  g.rows = sorted;
  g.row_div = (int)k;
  g.tile_expert = tile_expert;
  g.meta = meta;
  g.tab0 = w_gate;
  g.tab1 = w_up;
  g.ldb = I;
  g.c = inter_rows;
  g.ldc = I;
  g.N = I;
  g.K = H;
  const bool vec = aligned(x, 16) && H % 4 == 0 && I % 4 == 0;
  rc = f32_launch<false, true, true>(g, L.max_tiles, vec, st, "ccq_moe_f32_ffn gate/up");
  if (rc) return rc;
  F32GP d = {};
  d.a = inter_rows;
  d.lda = I;
  d.rows = sorted;
  d.row_div = 1;
  d.tile_expert = tile_expert;
  d.meta = meta;
  d.tab0 = w_down;
  d.ldb = H;
  d.c = rows;
  d.ldc = H;
  d.N = H;
  d.K = I;
  rc = f32_launch<false, false, true>(d, L.max_tiles, vec, st, "ccq_moe_f32_ffn down");
  if (rc) return rc;
  return launch_combine(rows, CCQ_F32, weights, ids, E, y, y_dtype, T, k, H, st, shared, shared_gate);
}
