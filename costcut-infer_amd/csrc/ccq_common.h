// Shared device/host helpers for libccq_hip (gfx950 / CDNA4).
//
// Conventions of the C ABI (declared in include/ccq.h):
//   * every entry point returns int: 0 ok, <0 argument error (message in
//     ccq_last_error()), >0 a hipError_t from a launch;
//   * all buffers are caller-owned device pointers; launches are ordered on
//     the caller's stream (a hipStream_t passed as void*); nothing allocates.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/ccq.h"

namespace ccq {

// ---------------------------------------------------------------- errors --
void set_error(const char* fmt, ...);
int arg_error(const char* fmt, ...);           // sets message, returns CCQ_EINVAL
int launch_status(const char* what);           // hipGetLastError -> code

// Events for the next kernel launched through launch() on this thread
// (ccq_launch_timer): hipExtLaunchKernel records them when that kernel
// starts and ends executing, so their elapsed time is the kernel's own
// duration.  take_launch_timer returns the pair and clears it.
struct LaunchTimer {
  hipEvent_t start, stop;
};
LaunchTimer take_launch_timer();

template <typename... KArgs, typename... Args>
inline void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t lds_bytes, hipStream_t st,
                   Args... args) {
  const LaunchTimer t = take_launch_timer();
  if (t.start != nullptr)
    hipExtLaunchKernelGGL(kernel, grid, block, lds_bytes, st, t.start, t.stop, 0u, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds_bytes, st, args...);
}

#define CCQ_REQUIRE(cond, ...)                                  \
  do {                                                          \
    if (!(cond)) return ::ccq::arg_error(__VA_ARGS__);          \
  } while (0)

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
// workgroups for a grid-stride loop over n items: at least 1, at most 65536
inline int grid_for(int64_t n, int block) {
  const int64_t g = cdiv(n, block);
  return (int)(g < 65536 ? (g < 1 ? 1 : g) : 65536);
}
__host__ __device__ inline int64_t imin64(int64_t a, int64_t b) { return a < b ? a : b; }

// ----------------------------------------------------------- vector types --
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8;

// --------------------------------------------------------- scalar codecs --
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  _Float16 h;
  uint16_t v = (uint16_t)b;
  __builtin_memcpy(&h, &v, 2);
  return (float)h;
}

// float -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two floats -> packed bf16 bits (a low, b high), round to nearest even:
// gfx950's v_cvt_pk_bf16_f32 (equal to f32_to_bf16_bits for every non-NaN
// float).
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
__device__ __forceinline__ uint32_t bf16x2_bits(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), bf16x2));
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;
  uint16_t v;
  __builtin_memcpy(&v, &h, 2);
  return v;
}

// e4m3fn byte -> float (exact).  exp==0: m*2^-9; exp==15,m==7: NaN.
__device__ __forceinline__ float fp8_e4m3_to_f32(uint32_t b) {
  uint32_t s = (b & 0x80u) << 24;
  uint32_t e = (b >> 3) & 0xFu;
  uint32_t m = b & 0x7u;
  if (e == 0) {
    float v = (float)m * 0.001953125f;  // m / 8 * 2^-6
    return __uint_as_float(__float_as_uint(v) | s);
  }
  if (e == 15 && m == 7) return __uint_as_float(0x7fc00000u | s);
  return __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
}

// float -> e4m3fn with round-to-nearest-even, saturating to +-448, NaN->0x7F.
__device__ __forceinline__ uint32_t f32_to_fp8_rne(float v) {
  uint32_t u = __float_as_uint(v);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return 0x7Fu;
  if (a >= 0x43e00000u) return sign | 0x7Eu;            // >= 448
  if (a < 0x3c800000u) {                                 // < 2^-6: subnormal grid m*2^-9
    float t = __uint_as_float(a) * 512.0f;               // exact scaling
    float fl = floorf(t);
    float fr = t - fl;
    uint32_t m = (uint32_t)fl;
    if (fr > 0.5f || (fr == 0.5f && (m & 1u))) m += 1;
    return sign | m;                                     // m == 8 is 0x08 = 2^-6
  }
  // normal: keep 3 mantissa bits, RNE on the 20 dropped bits
  uint32_t e = (a >> 23) - 120u;                         // e4m3 exponent code 1..15
  uint32_t mant = (a >> 20) & 7u;
  uint32_t rest = a & 0xFFFFFu;
  uint32_t code = (e << 3) | mant;
  if (rest > 0x80000u || (rest == 0x80000u && (mant & 1u))) code += 1;
  if (code > 0x7Eu) code = 0x7Eu;
  return sign | code;
}

// ---------------------------------------------------------- MX decoders --
// E8M0 scale byte -> float: 2^(e-127); e = 0 -> 0 and e = 255 -> NaN, as
// the reference's mx_e8m0_to_float (quant/kernels.py:240-256).
__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
  return e == 0u ? 0.f : (e == 255u ? __int_as_float(0x7fc00000) : __int_as_float((int)(e << 23)));
}

typedef _Float16 mx_h2 __attribute__((ext_vector_type(2)));

// Columns 8w..8w+7 of one 32-bit word of the reference's 4-bit codes (low
// nibble = even column; table 0, .5, 1, 1.5, -0, -.5, -1, -1.5 on code & 7,
// quant/mx.py:80), as float32: one v_perm_b32 per 4 codes picks the f16
// high bytes of the table's values (their low bytes are all zero), then
// v_cvt_f32_f16.
__device__ __forceinline__ void mx4_word(uint32_t w, float (&v)[8]) {
  constexpr uint32_t kLutLo = 0x3E3C3800u;  // f16 high bytes of 0, .5, 1, 1.5
  constexpr uint32_t kLutHi = 0xBEBCB880u;  // and of -0, -.5, -1, -1.5
  const uint32_t e = __builtin_amdgcn_perm(kLutHi, kLutLo, w & 0x07070707u);         // even columns
  const uint32_t o = __builtin_amdgcn_perm(kLutHi, kLutLo, (w >> 4) & 0x07070707u);  // odd columns
  const uint32_t sel[4] = {0x040C000Cu, 0x050C010Cu, 0x060C020Cu, 0x070C030Cu};
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const mx_h2 hv = __builtin_bit_cast(mx_h2, __builtin_amdgcn_perm(o, e, sel[b]));
    v[2 * b] = (float)hv.x;
    v[2 * b + 1] = (float)hv.y;
  }
}

// ------------------------------------- decoded-weight MFMA linear (host) --
// y[M, N] = x[M, K] @ W[N, K]^T on bf16 MFMA with the weights decoded in
// registers (ccq_wmfma.hip).  fmt: WQ_FP8_ROW e4m3 codes with a float32
// scale per output row; WQ_INT8_ROW int8 codes, float32 row scale;
// WQ_MXFP8 e4m3 codes with E8M0 group scales [N, K / G]; WQ_MXFP4 the
// reference's 4-bit codes (two per byte) with optional E8M0 group scales and
// the factor scale2 on each sum.  Returns 0 or a launch status, or -1 when
// the shape or alignment is not one the kernel takes (the caller then runs
// its own kernel); nothing is launched in that case.
enum WqFmt { WQ_FP8_ROW = 0, WQ_INT8_ROW = 1, WQ_MXFP8 = 2, WQ_MXFP4 = 3 };
int wq_mfma_linear(int fmt, const float* x, const uint8_t* w, const void* scale, int group_size, float scale2,
                   float* y, int64_t M, int64_t K, int64_t N, hipStream_t stream, const char* name);

// ------------------------------ expert schedule and combine (host side) --
// ccq_route.hip: the expert-sorted schedule of ccq_moe_align (scratch: the
// per-chunk tables of the many-workgroup form, align_scratch_bytes; without
// it larger batches take the one-workgroup kernel) and the weighted combine
// of ccq_moe_combine (rows float32 or bf16; shared: the shared expert's
// output, added after the routed sum).
int launch_align(const int64_t* ids, int64_t n, int64_t E, int64_t tile_m, int32_t* sorted_ids,
                 int32_t* tile_expert, int32_t* meta, int32_t* counts, hipStream_t st, void* scratch = nullptr,
                 size_t scratch_bytes = 0);
size_t align_scratch_bytes(int64_t n, int64_t E);
int launch_combine(const void* rows, int rows_dtype, const float* wts, const int64_t* ids, int64_t E, void* y,
                   int y_dtype, int64_t T, int64_t k, int64_t H, hipStream_t st, const float* shared = nullptr,
                   float shared_gate = 0.f);

// ------------------------------- schedule + activation side work (host) --
// Work on the layer input that runs beside a schedule, 16 threads per (row
// r < M, 128-column group g < KT): ALIGN_SIDE_SUMS, out[r * ldo + g] = the
// float32 sum, in a fixed order, of the group's 128 activations (x bf16 or
// f16, rows 16-byte aligned).  launch_align_side (ccq_route.hip) builds the
// schedule as launch_align does and, when the schedule has a one-workgroup
// launch (the mid-size kernel or the chunked plan), runs the side work on
// further workgroups of that launch (done = true); otherwise it launches
// nothing of it (done = false).  (The FP8 activation quantizer beside the
// chunked plan measured slower than its own launch: 43.7 against 16.5 +
// 20.5 µs at 2048 x 7168.)
enum AlignSideKind { ALIGN_SIDE_NONE = 0, ALIGN_SIDE_SUMS = 1 };
struct AlignSide {
  int kind;
  const void* x;
  int x_dtype;
  int64_t ldx, M, KT;
  float* out;
  int64_t ldo;
};
int launch_align_side(const int64_t* ids, int64_t n, int64_t E, int64_t tile_m, int32_t* sorted_ids,
                      int32_t* tile_expert, int32_t* meta, int32_t* counts, hipStream_t st, void* scratch,
                      size_t scratch_bytes, const AlignSide& side, bool& done);

// --------------------------------------------------------- wave helpers --
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

template <typename T>
__device__ __forceinline__ T wave_shfl_xor(T v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// ------------------------------------------------ LDS DMA pipeline pieces --
// Byte offset of a __shared__ object inside the workgroup's LDS.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// Global -> LDS without registers: lane l copies 16 (4) bytes from
// base + voff into LDS at lds + 16*l (4*l).  base and lds are wave-uniform;
// completion is counted by vmcnt.  Issued as inline assembly so that the
// compiler adds no waits of its own for the LDS it writes: the pipelines
// below order these copies with explicit wait_vmcnt + barrier.
// The compiler's hazard recognizer does not look into inline assembly, so
// the s_nop 4 provides the wait states the load needs after the instructions
// the compiler places right before it: a VALU write of the base SGPRs
// (v_readfirstlane, 5 wait states before a VMEM read of them) and the SALU
// write of M0 (1 wait state before an LDS DMA).
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t u = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u), hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return (const void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(uniform_ptr(base)), "{m0}"(lds) : "memory");
}
// The same copy marked non-temporal (nt), for data read once (weight
// streams), so it does not push reused data (activation tiles) out of L2.
__device__ __forceinline__ void dma16_nt(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(uniform_ptr(base)), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(uniform_ptr(base)), "{m0}"(lds) : "memory");
}

// Global -> VGPR 16-byte load of p + OFF issued as inline assembly, so that
// the compiler adds no wait of its own for it (it counts only the loads it
// issues itself): the caller waits with wait_vmcnt_tied, whose "+v"
// operands keep every use of the registers after that wait.  The address is
// a VGPR pair; VMEM reads of VGPRs written by VALU need no wait states.
// The load is marked non-temporal (nt): for data read once, such as weight
// streams.
template <int OFF>
__device__ __forceinline__ void gload16_nt(u32x4& dst, const void* p) {
  static_assert(OFF >= 0 && OFF < 4096, "13-bit signed immediate offset");
  asm volatile("global_load_dwordx4 %0, %1, off offset:%2 nt" : "=v"(dst) : "v"(p), "n"(OFF));
}

// Lane id computed where it is used: the compiler cannot hoist inline
// assembly out of a loop, so values derived from it are not kept live (in
// registers or spilled) across the loop.
__device__ __forceinline__ int lane_id_here() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// s_waitcnt vmcnt(N) that the compiler sees as producing the four register
// quads of one gload16 batch.
template <int N>
__device__ __forceinline__ void wait_vmcnt_tied(u32x4& a, u32x4& b, u32x4& c, u32x4& d) {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(N) : "memory");
}

// Wait until at most N vector-memory operations of this wave are in flight.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier that does not wait for outstanding global loads (the
// __syncthreads fence would drain the whole pipeline); LDS reads of this
// wave are completed first, so a slot may be refilled after the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Workgroups are dispatched round-robin over the 8 XCDs (linear id b runs on
// XCD b % 8).  Renumber ids 0..n-1 so that each XCD works through one
// contiguous range: neighbouring logical ids (for instance the column blocks
// of one row tile) then share that XCD's L2.
__device__ __forceinline__ int xcd_remap(int b, int n) {
  const int q = n >> 3, r = n & 7, x = b & 7;
  return x * q + (x < r ? x : r) + (b >> 3);
}

// Wait for this wave's copies of one k-step: n (wave-uniform) = copies the
// wave issues per k-step, N = the largest such count in the kernel.
template <int N>
__device__ __forceinline__ void wait_stage(int n) {
  if constexpr (N > 0) {
    if (n == N) {
      wait_vmcnt<N>();
      return;
    }
    wait_stage<N - 1>(n);
  } else {
    wait_vmcnt<0>();
  }
}

// Row reductions (sum, or max with MAX) over the 32 lanes of each half-wave
// for 32 values per lane, value r of a lane belonging to row r: a butterfly
// that halves the list at every step, so lane l ends with row l & 31.
template <bool MAX>
__device__ __forceinline__ float half_wave_row_reduce(float (&v)[32], int c32) {
#pragma unroll
  for (int m = 1, n = 32; m < 32; m <<= 1, n >>= 1) {
    const bool up = (c32 & m) != 0;
#pragma unroll
    for (int j = 0; j < n / 2; ++j) {
      const float keep = up ? v[2 * j + 1] : v[2 * j];
      const float send = up ? v[2 * j] : v[2 * j + 1];
      const float other = __shfl_xor(send, m, 64);
      v[j] = MAX ? fmaxf(keep, other) : keep + other;
    }
  }
  return v[0];
}

}  // namespace ccq
