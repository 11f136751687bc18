// Routing: top-k selection + softmax, expert-sorted tile schedule, combine.
//
// topk        reference python/ccut/blocks/moe.py:46-68
// topk_softmax reference python/ccut/blocks/moe.py:71-89
// route_experts reference python/ccut/blocks/moe.py:92-119 (norm_topk=0)
// token grouping reference python/ccut/blocks/moe.py:163-173,
//               python/ccut/models/generic.py:366-378
#include "ccq_common.h"
#include "ccq_topk.h"

#include <math.h>

namespace ccq {

constexpr int kMaxE = 1024;      // experts per row held in registers (16 per lane)
constexpr int kMaxK = 16;

// One wave per token row (topk_row), 4 rows per workgroup.
template <int PER>
__global__ __launch_bounds__(256) void topk_softmax_kernel(const float* __restrict__ logits,
                                                           float* __restrict__ weights,
                                                           int64_t* __restrict__ ids, int64_t T, int E,
                                                           int k, int mode) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= T) return;
  float w;
  int id;
  topk_row<PER>(logits + row * E, E, k, mode, w, id);
  if (lane < k) {
    weights[row * k + lane] = w;
    ids[row * k + lane] = id;
  }
}

// ----------------------------------------------------------------------------
// moe_align: one workgroup of 16 waves; wave w owns the contiguous segment
// [w*seg, (w+1)*seg) of the flat assignments, so "segment order, then order
// inside a segment" is the global order.  Stable ranks inside a 64-lane chunk
// come from ballot key matching (no atomics decide any position).
// ----------------------------------------------------------------------------
constexpr int kAlignWaves = 16;
constexpr int kIdCache = 32768;  // assignments whose expert ids are cached in LDS (int16)

struct AlignSmem {
  int16_t idc[kIdCache];
  int cnt[kMaxE];
  int first[kMaxE];
  int rank[kMaxE];
  int base[kMaxE];
  int inv[kMaxE];
  int wave_off[kAlignWaves][kMaxE];
  int wave_flags[kAlignWaves];
  int nactive;
};

__device__ __forceinline__ uint64_t match_key(int key, bool valid, int nbits) {
  uint64_t same = __ballot(valid);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (key >> b) & 1;
    const uint64_t bal = __ballot(valid && bit);
    same &= bit ? bal : ~bal;
  }
  return valid ? same : 0ull;
}

// The padding (-1) after each active expert's rows and the tile -> expert
// map, for a workgroup of nw waves and at most 64 nw active experts.  Lane l
// of wave w looks up rank w + nw l once (its expert, first padding slot,
// padding count, first tile and tile count); the wave then walks its ranks,
// taking each one's values from that lane, and its lanes store the rank's
// padding slots and tile entries side by side.  inv[r] = expert of rank r,
// base / cnt by expert.  No barrier.
__device__ void fill_padding_and_tiles(int nactive, int tile_m, const int* inv, const int* base, const int* cnt,
                                       int32_t* __restrict__ sorted_ids, int32_t* __restrict__ tile_expert) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int r = w + nw * lane;
  int e = 0, pad0 = 0, npad = 0, t0 = 0, nt = 0;
  if (r < nactive) {
    e = inv[r];
    const int b = base[e], c = cnt[e];
    nt = (c + tile_m - 1) / tile_m;
    pad0 = b + c;
    npad = nt * tile_m - c;
    t0 = b / tile_m;
  }
  const int nr = nactive > w ? (nactive - w + nw - 1) / nw : 0;  // ranks of this wave, <= 64
  for (int i = 0; i < nr; ++i) {
    const int ei = __builtin_amdgcn_readlane(e, i), p0 = __builtin_amdgcn_readlane(pad0, i);
    const int np = __builtin_amdgcn_readlane(npad, i), ti = __builtin_amdgcn_readlane(t0, i);
    const int nti = __builtin_amdgcn_readlane(nt, i);
    for (int j = lane; j < np; j += 64) sorted_ids[p0 + j] = -1;
    for (int j = lane; j < nti; j += 64) tile_expert[ti + j] = ei;
  }
}

// Thread gt of the side work (AlignSide), the row group sums: 16 lanes per
// (row, group), 8 activations per lane summed in order, then across the 16
// lanes by butterfly -- the arithmetic of row_group_sums_kernel (ccq_w4.hip).
__device__ void align_side_work(const AlignSide& s, int64_t gt) {
  const int64_t g = gt >> 4;
  const int part = threadIdx.x & 15;
  const bool ok = g < s.M * s.KT;
  // (32-bit division: M * KT < 2^31, checked where the side work is set up)
  const int64_t row = ok ? (int64_t)((uint32_t)g / (uint32_t)s.KT) : 0, kt = ok ? g - row * s.KT : 0;
  float acc = 0.f;
  if (ok) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(s.x) + row * s.ldx +
                                                    kt * 128 + part * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t b = (v[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
      acc += s.x_dtype == CCQ_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
    }
  }
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) acc += __shfl_xor(acc, off, 64);
  if (ok && part == 0) s.out[row * s.ldo + kt] = acc;
}

__global__ __launch_bounds__(1024) void moe_align_kernel(const int64_t* __restrict__ ids, int n, int E,
                                                         int tile_m, int32_t* __restrict__ sorted_ids,
                                                         int32_t* __restrict__ tile_expert,
                                                         int32_t* __restrict__ meta,
                                                         int32_t* __restrict__ counts_out) {
  __shared__ AlignSmem sm;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  for (int e = tid; e < E; e += 1024) {
    sm.cnt[e] = 0;
    sm.first[e] = 0x7fffffff;
  }
  for (int e = tid; e < kAlignWaves * E; e += 1024) (&sm.wave_off[0][0])[(e / E) * kMaxE + e % E] = 0;
  // the expert id of every assignment, read once (8 loads in flight per
  // thread) into LDS; -1 for ids outside [0, E)
  const bool cached = n <= kIdCache;
  if (cached) {
    for (int a0 = tid; a0 < n; a0 += 8 * 1024) {
      int64_t v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int a = a0 + u * 1024;
        v[u] = a < n ? ids[a] : -1;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int a = a0 + u * 1024;
        if (a < n) sm.idc[a] = (int16_t)((v[u] >= 0 && v[u] < E) ? v[u] : -1);
      }
    }
  }
  auto expert_of = [&](int a) -> int {
    if (cached) return sm.idc[a];
    const int64_t v = ids[a];
    return (v >= 0 && v < E) ? (int)v : -1;
  };
  __syncthreads();
  const int seg = (n + kAlignWaves - 1) / kAlignWaves;
  const int s0 = min(n, w * seg), s1 = min(n, s0 + seg);
  // pass A: per-expert counts (total and per wave) and first appearance
  for (int c = s0; c < s1; c += 64) {
    const int a = c + lane;
    const int e = a < s1 ? expert_of(a) : -1;
    const bool valid = e >= 0;
    const uint64_t same = match_key(e, valid, nbits);
    const uint64_t lower = same & ((1ull << lane) - 1ull);
    if (valid && lower == 0) {  // leader of its key in this chunk
      atomicAdd(&sm.cnt[e], __popcll(same));
      sm.wave_off[w][e] += __popcll(same);  // only this wave writes row w
      atomicMin(&sm.first[e], a);           // the leader is the lowest index
    }
  }
  __syncthreads();
  // pass B: expert ranks = order of first appearance
  int nflags = 0;
  for (int c = s0; c < s1; c += 64) {
    const int a = c + lane;
    bool flag = false;
    if (a < s1) {
      const int e = expert_of(a);
      flag = e >= 0 && sm.first[e] == a;
    }
    nflags += __popcll(__ballot(flag));
  }
  if (lane == 0) sm.wave_flags[w] = nflags;
  __syncthreads();
  {
    int before = 0;
    for (int i = 0; i < w; ++i) before += sm.wave_flags[i];
    for (int c = s0; c < s1; c += 64) {
      const int a = c + lane;
      const int e = a < s1 ? expert_of(a) : -1;
      const bool flag = e >= 0 && sm.first[e] == a;
      const uint64_t fl = __ballot(flag);
      if (flag) sm.rank[e] = before + __popcll(fl & ((1ull << lane) - 1ull));
      before += __popcll(fl);
    }
  }
  if (tid == 0) {
    int tot = 0;
    for (int i = 0; i < kAlignWaves; ++i) tot += sm.wave_flags[i];
    sm.nactive = tot;
  }
  __syncthreads();
  const int nactive = sm.nactive;
  for (int e = tid; e < E; e += 1024) {
    if (sm.cnt[e] > 0) sm.inv[sm.rank[e]] = e;
    counts_out[e] = sm.cnt[e];
  }
  // per-wave exclusive offsets inside each expert (wave order = global order)
  for (int e = tid; e < E; e += 1024) {
    int run = 0;
    for (int i = 0; i < kAlignWaves; ++i) {
      const int c = sm.wave_off[i][e];
      sm.wave_off[i][e] = run;
      run += c;
    }
  }
  __syncthreads();
  // padded bases in rank order (serial scan by one wave, nactive <= 1024)
  if (w == 0) {
    int carry = 0;
    for (int r0 = 0; r0 < nactive; r0 += 64) {
      const int r = r0 + lane;
      int p = 0;
      if (r < nactive) p = (int)cdiv(sm.cnt[sm.inv[r]], tile_m) * tile_m;
      int incl = p;
      for (int off = 1; off < 64; off <<= 1) {
        int o = __shfl_up(incl, off, 64);
        if (lane >= off) incl += o;
      }
      if (r < nactive) sm.base[sm.inv[r]] = carry + incl - p;
      carry += __shfl(incl, 63, 64);
    }
    if (lane == 0) {
      meta[0] = carry / tile_m;
      meta[1] = nactive;
    }
  }
  __syncthreads();
  // pass C: positions
  {
    for (int c = s0; c < s1; c += 64) {
      const int a = c + lane;
      const int e = a < s1 ? expert_of(a) : -1;
      const bool valid = e >= 0;
      const uint64_t same = match_key(e, valid, nbits);
      const int r = __popcll(same & ((1ull << lane) - 1ull));
      int off = 0;
      if (valid) off = sm.wave_off[w][e];
      __builtin_amdgcn_wave_barrier();
      if (valid) {
        sorted_ids[sm.base[e] + off + r] = a;
        if (r == 0) sm.wave_off[w][e] = off + __popcll(same);
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
  fill_padding_and_tiles(nactive, tile_m, sm.inv, sm.base, sm.cnt, sorted_ids, tile_expert);
}

// y[t, h] = sum_s w[t, s] * rows[t*k + s, h], slot order, float32.  Slots
// whose id is outside [0, E) (dropped by the schedule) contribute nothing.
// rows are float32 (RT = CCQ_F32) or bf16 (RT = CCQ_BF16); with VEC each
// thread takes 16 bytes of a row (4 or 8 columns) and, with yvec (y aligned
// for it), stores its columns in one vector store.  The ids, weights and
// rows of up to KMAX slots (8 or 16) are loaded before their FMAs (one
// memory round trip per KMAX slots, not one per slot); a dropped slot's row
// is read and not used.
// With shared (the shared expert's output [T, H] f32), the epilogue adds
// shared_gate * shared[t, h] to the sum, as shared_expert_add does
// (blocks/moe.py:177-179): the product rounded to float32, then the add.
template <int YT, int RT, bool VEC, int KMAX>
__global__ __launch_bounds__(256) void moe_combine_kernel(const void* __restrict__ rows,
                                                          const float* __restrict__ wts,
                                                          const int64_t* __restrict__ ids, int64_t E,
                                                          void* __restrict__ y, int64_t T, int k, int64_t H,
                                                          const float* __restrict__ shared, float shared_gate,
                                                          int yvec) {
  constexpr int CW = VEC ? (RT == CCQ_F32 ? 4 : 8) : 1;
  const int64_t t = blockIdx.y;
  const int64_t h = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * CW;
  if (h >= H) return;
  float acc[CW];
#pragma unroll
  for (int c = 0; c < CW; ++c) acc[c] = 0.f;
  for (int s0 = 0; s0 < k; s0 += KMAX) {  // chunks of KMAX slots, in slot order
    float wv[KMAX], r[KMAX][CW];
    bool ok[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (s0 + j < k) {
        const int64_t a = t * k + s0 + j;
        ok[j] = true;
        if (ids) {
          const int64_t e = ids[a];
          ok[j] = e >= 0 && e < E;
        }
        wv[j] = wts[a];
        if constexpr (RT == CCQ_F32) {
          const float* rp = reinterpret_cast<const float*>(rows) + a * H + h;
          if constexpr (VEC) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(rp);
#pragma unroll
            for (int c = 0; c < CW; ++c) r[j][c] = v[c];
          } else {
            r[j][0] = rp[0];
          }
        } else {
          const uint16_t* rp = reinterpret_cast<const uint16_t*>(rows) + a * H + h;
          if constexpr (VEC) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(rp);
#pragma unroll
            for (int c = 0; c < CW; ++c) r[j][c] = bf16_bits_to_f32((v[c >> 1] >> (16 * (c & 1))) & 0xFFFFu);
          } else {
            r[j][0] = bf16_bits_to_f32(rp[0]);
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < KMAX; ++j)
      if (s0 + j < k && ok[j])
#pragma unroll
        for (int c = 0; c < CW; ++c) acc[c] = fmaf(wv[j], r[j][c], acc[c]);
  }
  if (shared) {
#pragma clang fp contract(off)  // the product rounds on its own, as numpy's does
#pragma unroll
    for (int c = 0; c < CW; ++c) {
      const float g = shared_gate * shared[t * H + h + c];
      acc[c] = acc[c] + g;
    }
  }
  if constexpr (VEC) {
    if (yvec) {
      const int64_t o = t * H + h;
      if constexpr (YT == CCQ_F32) {
#pragma unroll
        for (int c = 0; c < CW; c += 4)
          *reinterpret_cast<f32x4*>((float*)y + o + c) = f32x4{acc[c], acc[c + 1], acc[c + 2], acc[c + 3]};
      } else {
        uint32_t wv2[CW / 2];
#pragma unroll
        for (int c = 0; c < CW; c += 2)
          wv2[c / 2] = YT == CCQ_BF16 ? (f32_to_bf16_bits(acc[c]) | (f32_to_bf16_bits(acc[c + 1]) << 16))
                                      : (f32_to_f16_bits(acc[c]) | (f32_to_f16_bits(acc[c + 1]) << 16));
        if constexpr (CW == 8)
          *reinterpret_cast<u32x4*>((uint16_t*)y + o) = u32x4{wv2[0], wv2[1], wv2[2], wv2[3]};
        else
          *reinterpret_cast<u32x2*>((uint16_t*)y + o) = u32x2{wv2[0], wv2[1]};
      }
      return;
    }
  }
#pragma unroll
  for (int c = 0; c < CW; ++c) {
    const int64_t o = t * H + h + c;
    if (YT == CCQ_F32)
      ((float*)y)[o] = acc[c];
    else if (YT == CCQ_BF16)
      ((uint16_t*)y)[o] = (uint16_t)f32_to_bf16_bits(acc[c]);
    else
      ((uint16_t*)y)[o] = (uint16_t)f32_to_f16_bits(acc[c]);
  }
}

template <int RT, bool VEC, int KMAX>
static void launch_combine_k(const void* rows, const float* wts, const int64_t* ids, int64_t E, void* y,
                             int y_dtype, int64_t T, int64_t k, int64_t H, hipStream_t st, const float* shared,
                             float sg) {
  constexpr int CW = VEC ? (RT == CCQ_F32 ? 4 : 8) : 1;
  const int64_t cols = VEC ? H / CW : H;
  dim3 grid((unsigned)cdiv(cols, 256), (unsigned)T);
  const int yvec = VEC && aligned(y, (size_t)CW * (y_dtype == CCQ_F32 ? 4 : 2)) ? 1 : 0;
  if (y_dtype == CCQ_F32)
    launch((moe_combine_kernel<CCQ_F32, RT, VEC, KMAX>), grid, dim3(256), 0, st, rows, wts, ids, E, y, T,
                       (int)k, H, shared, sg, yvec);
  else if (y_dtype == CCQ_BF16)
    launch((moe_combine_kernel<CCQ_BF16, RT, VEC, KMAX>), grid, dim3(256), 0, st, rows, wts, ids, E, y, T,
                       (int)k, H, shared, sg, yvec);
  else
    launch((moe_combine_kernel<CCQ_F16, RT, VEC, KMAX>), grid, dim3(256), 0, st, rows, wts, ids, E, y, T,
                       (int)k, H, shared, sg, yvec);
}

// slots per round trip: 8 for k <= 8 (the registers of 16 would halve the
// workgroups resident per compute unit), else 16
template <int RT, bool VEC>
static void launch_combine_v(const void* rows, const float* wts, const int64_t* ids, int64_t E, void* y,
                             int y_dtype, int64_t T, int64_t k, int64_t H, hipStream_t st, const float* shared,
                             float sg) {
  if (k <= 8)
    launch_combine_k<RT, VEC, 8>(rows, wts, ids, E, y, y_dtype, T, k, H, st, shared, sg);
  else
    launch_combine_k<RT, VEC, 16>(rows, wts, ids, E, y, y_dtype, T, k, H, st, shared, sg);
}

// rows_dtype CCQ_F32 or CCQ_BF16; shared optional (16-byte aligned for the
// vector forms).
int launch_combine(const void* rows, int rows_dtype, const float* wts, const int64_t* ids, int64_t E, void* y,
                   int y_dtype, int64_t T, int64_t k, int64_t H, hipStream_t st, const float* shared,
                   float shared_gate) {
  const bool sh_ok = !shared || aligned(shared, 16);
  if (rows_dtype == CCQ_BF16) {
    if (H % 8 == 0 && aligned(rows, 16) && sh_ok)
      launch_combine_v<CCQ_BF16, true>(rows, wts, ids, E, y, y_dtype, T, k, H, st, shared, shared_gate);
    else
      launch_combine_v<CCQ_BF16, false>(rows, wts, ids, E, y, y_dtype, T, k, H, st, shared, shared_gate);
  } else {
    if (H % 4 == 0 && aligned(rows, 16) && sh_ok)
      launch_combine_v<CCQ_F32, true>(rows, wts, ids, E, y, y_dtype, T, k, H, st, shared, shared_gate);
    else
      launch_combine_v<CCQ_F32, false>(rows, wts, ids, E, y, y_dtype, T, k, H, st, shared, shared_gate);
  }
  return launch_status("moe_combine");
}

// ----------------------------------------------------------------------------
// moe_align for large batches, over many workgroups: the same schedule as
// moe_align_kernel.  The assignments are cut into chunks of kChunk; a chunk
// is one workgroup of 4 waves, wave w owning the contiguous quarter
// [w*kChunk/4, (w+1)*kChunk/4) in 64-lane steps, so "chunk, wave, step,
// lane" order is the global order.
//  1. align_chunk_count: per chunk and expert, the count and the first index;
//  2. align_plan (one workgroup): totals, expert order by first appearance,
//     padded bases, meta / counts / tile_expert and the padding entries;
//  3. align_chunk_scatter: each assignment's slot = base + the counts of
//     the earlier chunks + offset of its wave in the chunk + rank among
//     equal ids before it.
// The scratch holds two [chunks][E] tables.
// ----------------------------------------------------------------------------
constexpr int kChunk = 1024;

// Chunk id-match ranks of one 64-lane step: lanes with equal expert ids.
__device__ __forceinline__ uint64_t step_match(const int64_t* ids, int a, int n, int E, int nbits, int& e) {
  const int64_t v = a < n ? ids[a] : -1;
  e = (v >= 0 && v < E) ? (int)v : -1;
  return match_key(e, e >= 0, nbits);
}

__global__ __launch_bounds__(256) void align_chunk_count_kernel(const int64_t* __restrict__ ids, int n, int E,
                                                                int32_t* __restrict__ ccnt,
                                                                int32_t* __restrict__ cfirst) {
  __shared__ int cnt[kMaxE], first[kMaxE];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, c = blockIdx.x;
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  for (int e = tid; e < E; e += 256) {
    cnt[e] = 0;
    first[e] = 0x7fffffff;
  }
  __syncthreads();
  const int q0 = c * kChunk + w * (kChunk / 4);
  for (int s = 0; s < kChunk / 4; s += 64) {
    const int a = q0 + s + lane;
    int e;
    const uint64_t same = step_match(ids, a, n, E, nbits, e);
    if (e >= 0 && (same & ((1ull << lane) - 1ull)) == 0) {  // lowest lane of its id
      atomicAdd(&cnt[e], __popcll(same));
      atomicMin(&first[e], a);
    }
  }
  __syncthreads();
  for (int e = tid; e < E; e += 256) {
    ccnt[(int64_t)c * E + e] = cnt[e];
    cfirst[(int64_t)c * E + e] = first[e];
  }
}

__global__ __launch_bounds__(1024) void align_plan_kernel(int E, int nchunks, int tile_m,
                                                          const int32_t* __restrict__ ccnt,
                                                          int32_t* __restrict__ cfirst, int32_t* __restrict__ sorted_ids,
                                                          int32_t* __restrict__ tile_expert, int32_t* __restrict__ meta,
                                                          int32_t* __restrict__ counts_out, const AlignSide side) {
  if (blockIdx.x > 0) {  // launched only with side work to run beside the plan
    align_side_work(side, (int64_t)(blockIdx.x - 1) * 1024 + threadIdx.x);
    return;
  }
  __shared__ int cnt[kMaxE], base[kMaxE], inv[kMaxE];
  __shared__ __align__(16) int key[kMaxE];  // first appearance, INT_MAX for unused experts
  __shared__ int nactive;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int e = tid; e < E; e += 1024) {  // loads only, 16 chunks in flight
    int run = 0, f = 0x7fffffff;
    for (int c0 = 0; c0 < nchunks; c0 += 16) {
      int x[16], y[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const bool in = c0 + u < nchunks;
        x[u] = in ? ccnt[(int64_t)(c0 + u) * E + e] : 0;
        y[u] = in ? cfirst[(int64_t)(c0 + u) * E + e] : 0x7fffffff;
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        run += x[u];
        f = min(f, y[u]);
      }
    }
    cnt[e] = run;
    key[e] = run > 0 ? f : 0x7fffffff;
    counts_out[e] = run;
  }
  for (int e = E + tid; e < ((E + 3) & ~3); e += 1024) key[e] = 0x7fffffff;  // whole 16-byte reads below
  __syncthreads();
  // order of first appearance: the number of used experts that appear
  // earlier (first appearances are distinct), four keys per LDS read
  for (int e = tid; e < E; e += 1024) {
    const int f = key[e];
    if (f != 0x7fffffff) {
      int r = 0;
      for (int e2 = 0; e2 < E; e2 += 4) {
        const int4 k4 = *reinterpret_cast<const int4*>(&key[e2]);
        r += (k4.x < f) + (k4.y < f) + (k4.z < f) + (k4.w < f);
      }
      inv[r] = e;
    }
  }
  if (w == 0) {
    int na = 0;
    for (int e = lane; e < E; e += 64) na += key[e] != 0x7fffffff ? 1 : 0;
    for (int off = 32; off >= 1; off >>= 1) na += __shfl_xor(na, off, 64);
    if (lane == 0) nactive = na;
  }
  __syncthreads();
  const int na = nactive;
  if (w == 0) {  // padded bases in rank order
    int carry = 0;
    for (int r0 = 0; r0 < na; r0 += 64) {
      const int r = r0 + lane;
      int p = 0;
      if (r < na) p = (int)cdiv(cnt[inv[r]], tile_m) * tile_m;
      int incl = p;
      for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(incl, off, 64);
        if (lane >= off) incl += o;
      }
      if (r < na) base[inv[r]] = carry + incl - p;
      carry += __shfl(incl, 63, 64);
    }
    if (lane == 0) {
      meta[0] = carry / tile_m;
      meta[1] = na;
    }
  }
  __syncthreads();
  for (int e = tid; e < E; e += 1024) cfirst[e] = cnt[e] > 0 ? base[e] : 0;  // row 0 of the table: the bases
  fill_padding_and_tiles(na, tile_m, inv, base, cnt, sorted_ids, tile_expert);
}

__global__ __launch_bounds__(256) void align_chunk_scatter_kernel(const int64_t* __restrict__ ids, int n, int E,
                                                                  const int32_t* __restrict__ ccnt,
                                                                  const int32_t* __restrict__ base,
                                                                  int32_t* __restrict__ sorted_ids) {
  __shared__ int woff[4][kMaxE];  // per wave: ids counted so far (then: offset of the wave's quarter)
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, c = blockIdx.x;
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  for (int i = tid; i < 4 * E; i += 256) woff[i / E][i % E] = 0;
  __syncthreads();
  const int q0 = c * kChunk + w * (kChunk / 4);
  for (int s = 0; s < kChunk / 4; s += 64) {  // per-wave counts of the quarter
    const int a = q0 + s + lane;
    int e;
    const uint64_t same = step_match(ids, a, n, E, nbits, e);
    if (e >= 0 && (same & ((1ull << lane) - 1ull)) == 0) woff[w][e] += __popcll(same);
  }
  __syncthreads();
  for (int e = tid; e < E; e += 256) {  // base + earlier chunks' counts, then the 4 quarters
    int run = base[e];
    for (int c0 = 0; c0 < c; c0 += 16) {
      int x[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = c0 + u < c ? ccnt[(int64_t)(c0 + u) * E + e] : 0;
#pragma unroll
      for (int u = 0; u < 16; ++u) run += x[u];
    }
    for (int q = 0; q < 4; ++q) {
      const int x = woff[q][e];
      woff[q][e] = run;
      run += x;
    }
  }
  __syncthreads();
  for (int s = 0; s < kChunk / 4; s += 64) {
    const int a = q0 + s + lane;
    int e;
    const uint64_t same = step_match(ids, a, n, E, nbits, e);
    const int r = __popcll(same & ((1ull << lane) - 1ull));
    int off = 0;
    if (e >= 0) off = woff[w][e];
    __builtin_amdgcn_wave_barrier();
    if (e >= 0) {
      sorted_ids[off + r] = a;
      if (r == 0) woff[w][e] = off + __popcll(same);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// The same schedule for small batches (decode: n <= 256 assignments) in one
// wave, with no barrier: lane l holds assignments l, 64 + l, 128 + l,
// 192 + l; ballots over the expert id bits match each assignment with the
// lanes of every chunk holding the same expert, which gives its rank among
// them (assignment order), its expert's count and whether it is the
// expert's first appearance; an exclusive scan over the first appearances,
// in assignment order, gives the padded bases.  Experts' bases and counts
// go through LDS (the lanes of an expert read its first lane's values).
constexpr int kSmallN = 256;

// NCH chunks of 64 assignments (n <= 64 NCH), NB expert id bits (E <= 2^NB):
// both compile-time, so the ballot matching is straight-line code
template <int NCH, int NB>
__global__ __launch_bounds__(64) void moe_align_small_kernel(const int64_t* __restrict__ ids, int n, int E,
                                                             int tile_m, int32_t* __restrict__ sorted_ids,
                                                             int32_t* __restrict__ tile_expert,
                                                             int32_t* __restrict__ meta,
                                                             int32_t* __restrict__ counts_out) {
  __shared__ int sbase[1 << NB];
  __shared__ int scnt[1 << NB];
  const int lane = threadIdx.x;
  for (int e = lane; e < E; e += 64) scnt[e] = 0;
  int key[NCH], rank[NCH], cnt[NCH];
  uint64_t vm[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int a = 64 * c + lane;
    const int64_t v = a < n ? ids[a] : -1;
    key[c] = (v >= 0 && v < E) ? (int)v : -1;
    vm[c] = __ballot(key[c] >= 0);
    rank[c] = 0;
    cnt[c] = 0;
  }
  const uint64_t lt = (1ull << lane) - 1ull;
#pragma unroll
  for (int d = 0; d < NCH; ++d) {
    uint64_t bd[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) bd[b] = __ballot(key[d] >= 0 && ((key[d] >> b) & 1));
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      uint64_t m = key[c] >= 0 ? vm[d] : 0ull;
#pragma unroll
      for (int b = 0; b < NB; ++b) m &= ((key[c] >> b) & 1) ? bd[b] : ~bd[b];
      cnt[c] += (int)__popcll(m);
      if (d < c) rank[c] += (int)__popcll(m);
      if (d == c) rank[c] += (int)__popcll(m & lt);
    }
  }
  // first appearances in assignment order: the experts' order and padded bases
  int carry = 0, nact = 0;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const bool first = key[c] >= 0 && rank[c] == 0;
    const int pd = first ? (cnt[c] + tile_m - 1) / tile_m * tile_m : 0;
    int incl = pd;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(incl, off, 64);
      if (lane >= off) incl += o;
    }
    if (first) {
      const int bs = carry + incl - pd;
      sbase[key[c]] = bs;
      scnt[key[c]] = cnt[c];
      for (int j = cnt[c]; j < pd; ++j) sorted_ids[bs + j] = -1;
      for (int t = bs / tile_m; t < (bs + pd) / tile_m; ++t) tile_expert[t] = key[c];
    }
    carry += __shfl(incl, 63, 64);
    nact += (int)__popcll(__ballot(first));
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the bases and counts above, before any lane reads them
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    if (key[c] >= 0) sorted_ids[sbase[key[c]] + rank[c]] = 64 * c + lane;
  for (int e = lane; e < E; e += 64) counts_out[e] = scnt[e];
  if (lane == 0) {
    meta[0] = carry / tile_m;
    meta[1] = nact;
  }
}

template <int NCH>
static void launch_align_small_nb(const int64_t* ids, int n, int E, int tile_m, int32_t* sorted_ids,
                                  int32_t* tile_expert, int32_t* meta, int32_t* counts, hipStream_t st) {
#define CCQ_ALS(NB)                                                                                          \
  launch((moe_align_small_kernel<NCH, NB>), dim3(1), dim3(64), 0, st, ids, n, E, tile_m, sorted_ids, tile_expert, \
         meta, counts)
  if (E <= 64)
    CCQ_ALS(6);
  else if (E <= 256)
    CCQ_ALS(8);
  else
    CCQ_ALS(10);
#undef CCQ_ALS
}

// n <= kSmallN, E <= 1024
static void launch_align_small(const int64_t* ids, int n, int E, int tile_m, int32_t* sorted_ids,
                               int32_t* tile_expert, int32_t* meta, int32_t* counts, hipStream_t st) {
  if (n <= 64)
    launch_align_small_nb<1>(ids, n, E, tile_m, sorted_ids, tile_expert, meta, counts, st);
  else if (n <= 128)
    launch_align_small_nb<2>(ids, n, E, tile_m, sorted_ids, tile_expert, meta, counts, st);
  else
    launch_align_small_nb<4>(ids, n, E, tile_m, sorted_ids, tile_expert, meta, counts, st);
}

// The same schedule for mid-size batches (kSmallN < n <= kMidN) in one
// workgroup of 16 waves: wave w holds chunks w*CPW .. w*CPW + CPW - 1 of 64
// assignments (lane l: assignment 64 c + l of its chunks), so wave order,
// then chunk order, then lane order is assignment order.  Per chunk, ballots
// over the NB expert id bits give every assignment the lanes with its expert
// and its rank among them; the chunk's lowest such lane adds the chunk's
// count to the wave's per-expert count in LDS (its old value, broadcast, is
// the count of that expert in the wave's earlier chunks) and keeps the
// expert's first appearance (LDS min).  An exclusive scan over the waves of
// every expert's counts, the first appearances ranked in assignment order
// (ballots, per-wave totals), a scan over the ranks of the padded sizes, and
// each assignment lands at base + earlier waves' count + its rank in the wave.
// Compile-time NB and CPW keep the matching straight-line code.
constexpr int kMidN = 8192;
constexpr int kMidStage = 16384;  // padded sorted-list length staged in LDS (64 KB)

// Workgroup 0 builds the schedule; workgroups 1.. (launched only with side
// work to run) take 1024 of its threads each.
template <int NB, int CPW>
__global__ __launch_bounds__(1024) void moe_align_mid_kernel(const int64_t* __restrict__ ids, int n, int E,
                                                             int tile_m, int32_t* __restrict__ sorted_ids,
                                                             int32_t* __restrict__ tile_expert,
                                                             int32_t* __restrict__ meta,
                                                             int32_t* __restrict__ counts_out,
                                                             const AlignSide side) {
  if (blockIdx.x > 0) {
    align_side_work(side, (int64_t)(blockIdx.x - 1) * 1024 + threadIdx.x);
    return;
  }
  __shared__ int wcnt[kAlignWaves * (1 << NB)];  // [wave][expert]: counts, then exclusive offsets
  __shared__ int cnt[1 << NB], first[1 << NB], base[1 << NB], inv[1 << NB], tstart[1 << NB];
  __shared__ int wtot[kAlignWaves];
  __shared__ int stage[kMidStage];  // the padded sorted list, when it fits
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int key[CPW];
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const int a = (w * CPW + c) * 64 + lane;
    const int64_t v = a < n ? ids[a] : -1;
    key[c] = (v >= 0 && v < E) ? (int)v : -1;
  }
  for (int i = tid; i < kAlignWaves * E; i += 1024) wcnt[(i / E) * (1 << NB) + i % E] = 0;
  for (int e = tid; e < E; e += 1024) first[e] = 0x7fffffff;
  __syncthreads();

  // pass A: rank of each assignment among the wave's assignments of its expert
  const uint64_t lt = (1ull << lane) - 1ull;
  int pos[CPW];
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const int e = key[c];
    const bool valid = e >= 0;
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const uint64_t bb = __ballot(valid && ((e >> b) & 1));
      m &= ((e >> b) & 1) ? bb : ~bb;
    }
    m = valid ? m : 0ull;
    const int r = (int)__popcll(m & lt);
    int old = 0;
    if (valid && r == 0) {
      old = atomicAdd(&wcnt[w * (1 << NB) + e], (int)__popcll(m));
      atomicMin(&first[e], (w * CPW + c) * 64 + lane);
    }
    old = __shfl(old, valid ? (int)__builtin_ctzll(m) : lane, 64);
    pos[c] = old + r;
  }
  __syncthreads();

  // per-expert exclusive offsets over the waves; first appearances per wave
  for (int e = tid; e < E; e += 1024) {
    int run = 0;
#pragma unroll
    for (int i = 0; i < kAlignWaves; ++i) {
      const int c = wcnt[i * (1 << NB) + e];
      wcnt[i * (1 << NB) + e] = run;
      run += c;
    }
    cnt[e] = run;
    counts_out[e] = run;
  }
  uint64_t fl[CPW];
  int nfl = 0;
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const int a = (w * CPW + c) * 64 + lane;
    fl[c] = __ballot(key[c] >= 0 && first[key[c]] == a);
    nfl += (int)__popcll(fl[c]);
  }
  if (lane == 0) wtot[w] = nfl;
  __syncthreads();

  // experts in first-appearance order
  int before = 0, nactive = 0;
#pragma unroll
  for (int i = 0; i < kAlignWaves; ++i) {
    const int t = wtot[i];
    before += i < w ? t : 0;
    nactive += t;
  }
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    if ((fl[c] >> lane) & 1) inv[before + (int)__popcll(fl[c] & lt)] = key[c];
    before += (int)__popcll(fl[c]);
  }
  __syncthreads();

  // padded bases in rank order: wave w scans ranks 64 w .. 64 w + 63
  const int rk = 64 * w + lane;
  const int pd = rk < nactive ? (cnt[inv[rk]] + tile_m - 1) / tile_m * tile_m : 0;
  int incl = pd;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane == 63) wtot[w] = incl;  // every wave read the flag totals before the last barrier
  __syncthreads();
  int boff = 0, total = 0;
#pragma unroll
  for (int i = 0; i < kAlignWaves; ++i) {
    const int t = wtot[i];
    boff += i < w ? t : 0;
    total += t;
  }
  if (rk < nactive) {
    base[inv[rk]] = boff + incl - pd;
    tstart[rk] = (boff + incl - pd) / tile_m;
  }
  if (tid == 0) {
    meta[0] = total / tile_m;
    meta[1] = nactive;
  }
  const bool staged = total <= kMidStage;  // the same in every wave
  if (staged)
    for (int i = tid; i < total; i += 1024) stage[i] = -1;
  __syncthreads();

  if (staged) {
    // the list is assembled in LDS and written out in order: one workgroup's
    // scattered 4-byte stores to HBM would queue behind each other
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int e = key[c];
      if (e >= 0) stage[base[e] + wcnt[w * (1 << NB) + e] + pos[c]] = (w * CPW + c) * 64 + lane;
    }
    __syncthreads();
    for (int i = tid; i < total; i += 1024) sorted_ids[i] = stage[i];
    for (int t = tid; t < total / tile_m; t += 1024) {
      int lo = 0, hi = nactive - 1;  // the largest rank whose first tile is <= t
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tstart[mid] <= t)
          lo = mid;
        else
          hi = mid - 1;
      }
      tile_expert[t] = inv[lo];
    }
  } else {
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int e = key[c];
      if (e >= 0) sorted_ids[base[e] + wcnt[w * (1 << NB) + e] + pos[c]] = (w * CPW + c) * 64 + lane;
    }
    fill_padding_and_tiles(nactive, tile_m, inv, base, cnt, sorted_ids, tile_expert);
  }
}

// side.kind != ALIGN_SIDE_NONE: the side work on workgroups 1..
template <int CPW>
static void launch_align_mid_nb(const int64_t* ids, int n, int E, int tile_m, int32_t* sorted_ids,
                                int32_t* tile_expert, int32_t* meta, int32_t* counts, hipStream_t st,
                                const AlignSide& side) {
  const unsigned grid = 1u + (side.kind != ALIGN_SIDE_NONE ? (unsigned)cdiv(side.M * side.KT * 16, 1024) : 0u);
#define CCQ_ALM(NB)                                                                                          \
  launch((moe_align_mid_kernel<NB, CPW>), dim3(grid), dim3(1024), 0, st, ids, n, E, tile_m, sorted_ids,     \
         tile_expert, meta, counts, side)
  if (E <= 64)
    CCQ_ALM(6);
  else if (E <= 256)
    CCQ_ALM(8);
  else
    CCQ_ALM(10);
#undef CCQ_ALM
}

// kSmallN < n <= kMidN, E <= 1024
static void launch_align_mid(const int64_t* ids, int n, int E, int tile_m, int32_t* sorted_ids,
                             int32_t* tile_expert, int32_t* meta, int32_t* counts, hipStream_t st,
                             const AlignSide& side) {
  if (n <= 1024)
    launch_align_mid_nb<1>(ids, n, E, tile_m, sorted_ids, tile_expert, meta, counts, st, side);
  else if (n <= 2048)
    launch_align_mid_nb<2>(ids, n, E, tile_m, sorted_ids, tile_expert, meta, counts, st, side);
  else if (n <= 4096)
    launch_align_mid_nb<4>(ids, n, E, tile_m, sorted_ids, tile_expert, meta, counts, st, side);
  else
    launch_align_mid_nb<8>(ids, n, E, tile_m, sorted_ids, tile_expert, meta, counts, st, side);
}

size_t align_scratch_bytes(int64_t n, int64_t E) { return (size_t)2 * cdiv(n, kChunk) * E * 4; }

// side.kind != ALIGN_SIDE_NONE: the side work also runs, on extra
// workgroups of the one-workgroup launch (mid-size kernel or chunked plan;
// done = true), when the schedule has one; with the small and the generic
// kernels it is left to the caller (done = false)
static int launch_align_impl(const int64_t* ids, int64_t n, int64_t E, int64_t tile_m, int32_t* sorted_ids,
                             int32_t* tile_expert, int32_t* meta, int32_t* counts, hipStream_t st, void* scratch,
                             size_t scratch_bytes, const AlignSide& side, bool& done) {
  done = false;
  const int64_t nchunks = cdiv(n, kChunk);
  if (n <= kSmallN && E <= kMaxE) {  // decode batches: one wave
    launch_align_small(ids, (int)n, (int)E, (int)tile_m, sorted_ids, tile_expert, meta, counts, st);
    return launch_status("moe_align (small)");
  }
  if (n <= kMidN && E <= kMaxE) {  // one workgroup, straight-line matching
    launch_align_mid(ids, (int)n, (int)E, (int)tile_m, sorted_ids, tile_expert, meta, counts, st, side);
    done = side.kind != ALIGN_SIDE_NONE;
    return launch_status("moe_align (mid)");
  }
  // larger batches: three launches over many workgroups when there is
  // scratch for the per-chunk counts, else the generic one-workgroup kernel
  if (scratch == nullptr || scratch_bytes < align_scratch_bytes(n, E)) {
    launch(moe_align_kernel, dim3(1), dim3(1024), 0, st, ids, (int)n, (int)E, (int)tile_m, sorted_ids,
                       tile_expert, meta, counts);
    return launch_status("moe_align");
  }
  int32_t* ccnt = (int32_t*)scratch;
  int32_t* cfirst = ccnt + nchunks * E;
  launch(align_chunk_count_kernel, dim3((unsigned)nchunks), dim3(256), 0, st, ids, (int)n, (int)E, ccnt,
                     cfirst);
  const unsigned pgrid = 1u + (side.kind != ALIGN_SIDE_NONE ? (unsigned)cdiv(side.M * side.KT * 16, 1024) : 0u);
  launch(align_plan_kernel, dim3(pgrid), dim3(1024), 0, st, (int)E, (int)nchunks, (int)tile_m, ccnt, cfirst,
                     sorted_ids, tile_expert, meta, counts, side);
  done = side.kind != ALIGN_SIDE_NONE;
  launch(align_chunk_scatter_kernel, dim3((unsigned)nchunks), dim3(256), 0, st, ids, (int)n, (int)E, ccnt,
                     cfirst, sorted_ids);
  return launch_status("moe_align (chunked)");
}

int launch_align(const int64_t* ids, int64_t n, int64_t E, int64_t tile_m, int32_t* sorted_ids,
                 int32_t* tile_expert, int32_t* meta, int32_t* counts, hipStream_t st, void* scratch,
                 size_t scratch_bytes) {
  bool done = false;
  return launch_align_impl(ids, n, E, tile_m, sorted_ids, tile_expert, meta, counts, st, scratch, scratch_bytes,
                           AlignSide{}, done);
}

int launch_align_side(const int64_t* ids, int64_t n, int64_t E, int64_t tile_m, int32_t* sorted_ids,
                      int32_t* tile_expert, int32_t* meta, int32_t* counts, hipStream_t st, void* scratch,
                      size_t scratch_bytes, const AlignSide& side, bool& done) {
  done = false;
  const bool fits = side.kind != ALIGN_SIDE_NONE && side.M * side.KT * 16 < ((int64_t)1 << 31);
  return launch_align_impl(ids, n, E, tile_m, sorted_ids, tile_expert, meta, counts, st, scratch, scratch_bytes,
                           fits ? side : AlignSide{}, done);
}

}  // namespace ccq

using namespace ccq;

extern "C" int ccq_topk_softmax(const float* logits, float* weights, int64_t* ids, int64_t T, int64_t E, int64_t k,
                                int mode, void* stream) {
  CCQ_REQUIRE(T >= 0, "ccq_topk_softmax: T < 0");
  CCQ_REQUIRE(E >= 1 && E <= kMaxE, "ccq_topk_softmax: E=%lld outside [1, %d]", (long long)E, kMaxE);
  CCQ_REQUIRE(k >= 1 && k <= kMaxK && k <= E, "ccq_topk_softmax: k=%lld outside [1, min(%d, E)]", (long long)k,
              kMaxK);
  CCQ_REQUIRE(mode >= 0 && mode <= 4, "ccq_topk_softmax: mode=%d not in {0,1,2,3,4}", mode);
  if (T == 0) return 0;
  CCQ_REQUIRE(logits && weights && ids, "ccq_topk_softmax: null pointer");
  CCQ_REQUIRE(T <= (int64_t)4 * 0x7fffffff, "ccq_topk_softmax: T too large");
  const dim3 grid((unsigned)cdiv(T, 4));
  hipStream_t st = as_stream(stream);
  if (E <= 64)
    launch(topk_softmax_kernel<1>, grid, dim3(256), 0, st, logits, weights, ids, T, (int)E, (int)k, mode);
  else if (E <= 128)
    launch(topk_softmax_kernel<2>, grid, dim3(256), 0, st, logits, weights, ids, T, (int)E, (int)k, mode);
  else if (E <= 256)
    launch(topk_softmax_kernel<4>, grid, dim3(256), 0, st, logits, weights, ids, T, (int)E, (int)k, mode);
  else
    launch(topk_softmax_kernel<16>, grid, dim3(256), 0, st, logits, weights, ids, T, (int)E, (int)k,
                       mode);
  return launch_status("ccq_topk_softmax");
}

extern "C" int64_t ccq_moe_align_max_tiles(int64_t num_assignments, int64_t num_experts, int64_t tile_m) {
  if (num_assignments <= 0 || num_experts <= 0 || tile_m <= 0) return 0;
  return cdiv(num_assignments, tile_m) + (num_assignments < num_experts ? num_assignments : num_experts);
}

extern "C" int ccq_moe_align(const int64_t* ids, int64_t num_assignments, int64_t num_experts, int64_t tile_m,
                             int32_t* sorted_ids, int32_t* tile_expert, int32_t* meta, int32_t* counts,
                             void* stream) {
  CCQ_REQUIRE(num_assignments >= 0 && num_assignments <= 65536,
              "ccq_moe_align: num_assignments=%lld outside [0, 65536]", (long long)num_assignments);
  CCQ_REQUIRE(num_experts >= 1 && num_experts <= kMaxE, "ccq_moe_align: num_experts=%lld outside [1, %d]",
              (long long)num_experts, kMaxE);
  CCQ_REQUIRE(tile_m >= 1 && tile_m <= 4096, "ccq_moe_align: tile_m=%lld outside [1, 4096]", (long long)tile_m);
  CCQ_REQUIRE(meta && counts && (num_assignments == 0 || (ids && sorted_ids && tile_expert)),
              "ccq_moe_align: null pointer");
  return launch_align(ids, num_assignments, num_experts, tile_m, sorted_ids, tile_expert, meta, counts,
                      as_stream(stream), nullptr, 0);
}

extern "C" int ccq_moe_combine(const float* rows, const float* weights, void* y, int y_dtype, int64_t T, int64_t k,
                               int64_t H, void* stream) {
  CCQ_REQUIRE(T >= 0 && k >= 1 && H >= 0, "ccq_moe_combine: bad shape");
  CCQ_REQUIRE(y_dtype == CCQ_F32 || y_dtype == CCQ_BF16 || y_dtype == CCQ_F16, "ccq_moe_combine: bad y_dtype");
  CCQ_REQUIRE(T <= 65535, "ccq_moe_combine: T=%lld > 65535", (long long)T);
  if (T == 0 || H == 0) return 0;
  CCQ_REQUIRE(rows && weights && y, "ccq_moe_combine: null pointer");
  return launch_combine(rows, CCQ_F32, weights, nullptr, 0, y, y_dtype, T, k, H, as_stream(stream), nullptr, 0.f);
}

extern "C" int ccq_moe_combine_shared(const float* rows, const float* weights, const float* shared,
                                      float shared_gate, void* y, int y_dtype, int64_t T, int64_t k, int64_t H,
                                      void* stream) {
  CCQ_REQUIRE(T >= 0 && k >= 1 && H >= 0, "ccq_moe_combine_shared: bad shape");
  CCQ_REQUIRE(y_dtype == CCQ_F32 || y_dtype == CCQ_BF16 || y_dtype == CCQ_F16,
              "ccq_moe_combine_shared: bad y_dtype");
  CCQ_REQUIRE(T <= 65535, "ccq_moe_combine_shared: T=%lld > 65535", (long long)T);
  if (T == 0 || H == 0) return 0;
  CCQ_REQUIRE(rows && weights && shared && y, "ccq_moe_combine_shared: null pointer");
  return launch_combine(rows, CCQ_F32, weights, nullptr, 0, y, y_dtype, T, k, H, as_stream(stream), shared,
                        shared_gate);
}

// y += gate * shared (float32: the product rounded, then the add), in place
__global__ void shared_add_kernel(float* __restrict__ y, const float* __restrict__ s, float g, int64_t n) {
#pragma clang fp contract(off)  // no fused multiply-add
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    const float p = g * s[i];
    y[i] = y[i] + p;
  }
}

extern "C" int ccq_shared_expert_add(float* y, const float* shared, float shared_gate, int64_t n, void* stream) {
  CCQ_REQUIRE(n >= 0, "ccq_shared_expert_add: negative size");
  if (n == 0) return 0;
  CCQ_REQUIRE(y && shared, "ccq_shared_expert_add: null pointer");
  const int64_t g = cdiv(n, 256);
  launch(shared_add_kernel, dim3((unsigned)(g < 65536 ? g : 65536)), dim3(256), 0, as_stream(stream), y,
                     shared, shared_gate, n);
  return launch_status("ccq_shared_expert_add");
}
