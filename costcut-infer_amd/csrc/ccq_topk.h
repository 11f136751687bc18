// Top-k routing of one token row by one wave, shared by the routing kernel
// and the fused decode MoE kernel so that both select bit-identical experts
// and weights.
//
// topk         reference python/ccut/blocks/moe.py:46-68
// topk_softmax reference python/ccut/blocks/moe.py:71-89
// route_experts reference python/ccut/blocks/moe.py:92-119 (norm_topk=0)
#pragma once

#include "ccq_common.h"

#include <math.h>

namespace ccq {

// Cross-lane steps on the VALU: DPP moves within 16-lane rows and
// v_readlane across them (a shuffle through ds_bpermute costs an LDS round
// trip per step, and the selection below runs k of them per row).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ float lane_f(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}

// The maximum over the wave (fmaxf), in every lane.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f<0x124>(v));  // row_ror:4
  v = fmaxf(v, dpp_f<0x128>(v));  // row_ror:8: every lane holds its row's maximum
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
// The minimum over the wave, in every lane.
__device__ __forceinline__ int wave_min(int v) {
  v = min(v, dpp_i<0xB1>(v));
  v = min(v, dpp_i<0x4E>(v));
  v = min(v, dpp_i<0x124>(v));
  v = min(v, dpp_i<0x128>(v));
  const int a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  const int c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return min(min(a, b), min(c, d));
}

// The maximum over the wave of unsigned keys, in every lane (max with 0 as
// the DPP fill value folds each move into the max instruction).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)dpp_i<0xB1>((int)v));
  v = max(v, (uint32_t)dpp_i<0x4E>((int)v));
  v = max(v, (uint32_t)dpp_i<0x124>((int)v));
  v = max(v, (uint32_t)dpp_i<0x128>((int)v));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}

// numpy's pairwise float32 summation of n <= 16 values, value j held by lane
// j: below 8 a plain running sum in index order; otherwise 8 partial sums
// r[j] = a[j] (+ a[8+j] when n == 16) combined as
// ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), then the tail in order.  Returned in
// every lane.
__device__ inline float np_pairwise_sum16(float a, int n) {
  if (n < 8) {
    float res = 0.f;  // numpy starts from -0.0; identical for these (positive) inputs
    for (int i = 0; i < n; ++i) res += lane_f(a, i);
    return res;
  }
  const int whole = n - (n % 8);  // 8 or 16
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = lane_f(a, j) + (8 + j < whole ? lane_f(a, 8 + j) : 0.f);
  float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (int i = whole; i < n; ++i) res += lane_f(a, i);
  return res;
}

// numpy's maximum(a, b) for a constant b: NaN in a propagates (fmaxf would
// return b).
__device__ __forceinline__ float np_maximum(float a, float b) { return a != a ? a : fmaxf(a, b); }

// Routing of R token rows by one wave, row r at lr + r * stride.  Lane l
// holds columns l, l+64, ... (PER values, PER = ceil(E / 64) rounded up to
// 1, 2, 4 or 16); on return lanes j < k hold the weight and expert id of
// slot j of each row.  The R rows run interleaved (R > 1 only with one
// column per lane): each step below is a chain of cross-lane operations,
// and independent rows fill each other's latency.
template <int PER, int R>
__device__ __forceinline__ void topk_rows(const float* __restrict__ lr, int64_t stride, int E, int k, int mode,
                                          float (&w_out)[R], int (&id_out)[R]) {
  static_assert(R == 1 || PER == 1, "several rows per wave with one column per lane only");
  const int lane = lane_id();
  float v[R][PER];
  bool used[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) used[i] = lane + 64 * i >= E;  // out-of-range slots never selectable
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int i = 0; i < PER; ++i) v[r][i] = used[i] ? -INFINITY : lr[r * stride + lane + 64 * i];
  if (mode == 0) {
    // p = exp(x - max) / maximum(sum, 1e-30) in float32 (blocks/moe.py:80-81)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float m = -INFINITY;
#pragma unroll
      for (int i = 0; i < PER; ++i)
        if (!used[i]) m = fmaxf(m, v[r][i]);
      m = wave_max(m);
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < PER; ++i)
        if (!used[i]) {
          v[r][i] = expf(v[r][i] - m);
          s += v[r][i];
        }
      for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
      const float d = np_maximum(s, 1e-30f);
#pragma unroll
      for (int i = 0; i < PER; ++i)
        if (!used[i]) v[r][i] = v[r][i] / d;
    }
  }
  // k passes of "first value strictly greater than the running best" with the
  // best starting at -1e30 (ties -> lowest column; NaN never picked) select
  // the values > -1e30 in descending order, ties to the lowest column, and
  // fill the slots left over with (-1e30, -1).
  float my_v[R];
  int my_i[R];
  if constexpr (PER == 1) {
    // One column per lane: the same k passes on integer keys.  Eligible
    // values map to keys >= 1 in the same order (-0 keyed as +0, since the
    // float passes treat them as equal), the others to 0; a pass takes the
    // wave's largest key (DPP steps that fold into the max instructions),
    // the lowest lane holding it, and clears that lane.  A pass that finds
    // only zeros (nothing > -1e30 left) stores (-1e30, -1), as do all later
    // ones.
    uint32_t cur[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const bool elig = !used[0] && v[r][0] > -1.0e30f;
      const uint32_t u = __float_as_uint(v[r][0] == 0.f ? 0.f : v[r][0]);
      cur[r] = elig ? ((u & 0x80000000u) ? ~u : (u | 0x80000000u)) : 0u;
      my_v[r] = -1.0e30f;
      my_i[r] = -1;
    }
    for (int j = 0; j < k; ++j) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t m = wave_max_u32(cur[r]);
        const uint64_t eq = __ballot(cur[r] == m);
        const int L = m != 0u ? (int)__builtin_ctzll(eq) : -1;
        const float vL = lane_f(v[r][0], L & 63);
        my_v[r] = lane == j && L >= 0 ? vL : my_v[r];
        my_i[r] = lane == j ? L : my_i[r];
        cur[r] = lane == L ? 0u : cur[r];
      }
    }
  } else {
    const int r = 0;
  for (int j = 0; j < k; ++j) {
    float bv = -1.0e30f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int c = lane + 64 * i;
      if (!used[i] && v[r][i] > bv) {  // per lane columns are increasing
        bv = v[r][i];
        bi = c;
      }
    }
    const float m = wave_max(bv);
    if (m > -1.0e30f) {
      bi = wave_min(bv == m ? bi : 0x7fffffff);
      bv = lane_f(bv, bi & 63);  // the value at that column (+0 and -0 compare equal)
    } else {  // nothing > -1e30: reference stores (-1e30, -1)
      bi = -1;  // and its used[-1] = 1 marks the last column
      bv = -1.0e30f;
    }
    const int mark = bi >= 0 ? bi : E - 1;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (lane + 64 * i == mark) used[i] = true;
    if (lane == j) {
      my_v[r] = bv;
      my_i[r] = bi;
    }
  }
  }
  const bool mine = lane < k;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float w = my_v[r];  // modes 0 and 3: the selected values themselves
    if (mode == 1) {
      // v = vals - vals.max(); exp; / maximum(exp.sum(), 1e-30)  (blocks/moe.py:86-88);
      // the slots hold the values in descending order (fillers -1e30 last),
      // so the maximum is slot 0's
      const float m = lane_f(my_v[r], 0);
      const float e = mine ? expf(my_v[r] - m) : 0.f;
      const float d = np_maximum(np_pairwise_sum16(e, k), 1e-30f);
      w = e / d;
    } else if (mode == 2 || mode == 4) {
      // route_experts: exp(v - m) (norm_topk=1, m the largest selected value)
      // or exp(v) (norm_topk=0) over a float64 running sum, weights 0 when
      // the sum is not > 0 (blocks/moe.py:104-118).  The reference's m is a
      // float64 starting at -1e30, above the float32 slot filler -1e30f: a
      // row with nothing selected has exp(v - m) = 0 in every slot, so
      // weights 0.
      const float m = mode == 4 ? lane_f(my_v[r], 0) : 0.f;
      const float e = mine && (mode == 2 || m > -1.0e30f) ? expf(my_v[r] - m) : 0.f;
      double s = 0.0;
      for (int j = 0; j < k; ++j) s += (double)lane_f(e, j);
      w = s > 0.0 ? (float)((double)e / s) : 0.f;
    }
    w_out[r] = w;
    id_out[r] = my_i[r];
  }
}

template <int PER>
__device__ __forceinline__ void topk_row(const float* __restrict__ lr, int E, int k, int mode, float& w_out,
                                         int& id_out) {
  float w[1];
  int id[1];
  topk_rows<PER, 1>(lr, 0, E, k, mode, w, id);
  w_out = w[0];
  id_out = id[0];
}

}  // namespace ccq
