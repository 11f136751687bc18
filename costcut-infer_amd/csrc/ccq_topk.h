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

// Routing of one token row by one wave.  Lane l holds columns l, l+64, ...
// (PER values, PER = ceil(E / 64) rounded up to 1, 2, 4 or 16); after
// selection pass j, lane j holds slot j; on return lanes j < k hold the
// weight and expert id of slot j.  The code stays compact (a run-time loop
// over the k passes, no per-slot arrays): it runs on a handful of CUs, where
// a large body costs more in cold instruction fetches than it saves.
template <int PER>
__device__ __forceinline__ void topk_row(const float* __restrict__ lr, int E, int k, int mode, float& w_out,
                                         int& id_out) {
  const int lane = lane_id();
  float v[PER];
  bool used[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    int c = lane + 64 * i;
    v[i] = c < E ? lr[c] : -INFINITY;
    used[i] = c >= E;  // out-of-range slots never selectable
  }
  if (mode == 0) {
    // p = exp(x - max) / max(sum, 1e-30) in float32 (blocks/moe.py:80-81)
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (!used[i]) m = fmaxf(m, v[i]);
    m = wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (!used[i]) {
        v[i] = expf(v[i] - m);
        s += v[i];
      }
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
    const float d = np_maximum(s, 1e-30f);
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (!used[i]) v[i] = v[i] / d;
  }
  // k passes of "first value strictly greater than the running best" with the
  // best starting at -1e30 (ties -> lowest column; NaN never picked) select
  // the values > -1e30 in descending order, ties to the lowest column, and
  // fill the slots left over with (-1e30, -1).
  float my_v = 0.f;
  int my_i = 0;
  if constexpr (PER == 1) {
    // One column per lane: the same selection without k passes.  Eligible
    // values map to integer keys in the same order (-0 keyed as +0, since
    // the passes treat them as equal); ballots over the key bits find the
    // k-th largest key, the lanes above it and the lowest-column lanes equal
    // to it are the selection, and each selected lane's slot is the number
    // of selected lanes before it in (value desc, column asc) order.
    // Eligible keys are >= 1 (0 would be the NaN bit pattern 0xFFFFFFFF),
    // the others are 0, so every test against a threshold >= 1 below
    // excludes them.
    const bool elig = !used[0] && v[0] > -1.0e30f;
    const uint32_t u = __float_as_uint(v[0] == 0.f ? 0.f : v[0]);
    const uint32_t key = elig ? ((u & 0x80000000u) ? ~u : (u | 0x80000000u)) : 0u;
    const int ne = (int)__popcll(__ballot(elig));
    const int kk = ne < k ? ne : k;
    uint32_t th = 0;
    for (int b = 31; b >= 0; --b) {
      const uint32_t t = th | (1u << b);
      if ((int)__popcll(__ballot(key >= t)) >= kk) th = t;
    }
    uint64_t sel = __ballot(key > th);
    uint64_t eq = __ballot(key == th);
    for (int need = kk - (int)__popcll(sel); need > 0; --need) {
      const uint64_t low = eq & (~eq + 1ull);
      sel |= low;
      eq ^= low;
    }
    if (kk == 0) sel = 0;
    my_v = -1.0e30f;  // slots past the selection: (-1e30, -1)
    my_i = -1;
    for (uint64_t m = sel; m != 0; m &= m - 1) {
      const int L = (int)__builtin_ctzll(m);
      const uint32_t kL = (uint32_t)__builtin_amdgcn_readlane((int)key, L);
      const int slot = (int)__popcll(sel & __ballot(key > kL)) +
                       (int)__popcll(sel & __ballot(key == kL) & ((1ull << L) - 1ull));
      if (lane == slot) {
        my_v = lane_f(v[0], L);
        my_i = L;
      }
    }
  } else {
  for (int j = 0; j < k; ++j) {
    float bv = -1.0e30f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int c = lane + 64 * i;
      if (!used[i] && v[i] > bv) {  // per lane columns are increasing
        bv = v[i];
        bi = c;
      }
    }
    const float m = wave_max(bv);
    if (m > -1.0e30f) {
      if constexpr (PER == 1) {
        bi = (int)__builtin_ctzll(__ballot(bv == m));  // column = lane
      } else {
        bi = wave_min(bv == m ? bi : 0x7fffffff);
      }
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
      my_v = bv;
      my_i = bi;
    }
  }
  }
  const bool mine = lane < k;
  float w = my_v;  // modes 0 and 3: the selected values themselves
  if (mode == 1) {
    // v = vals - vals.max(); exp; / max(exp.sum(), 1e-30)  (blocks/moe.py:86-88)
    const float m = wave_max(mine ? my_v : -INFINITY);
    const float e = mine ? expf(my_v - m) : 0.f;
    const float d = np_maximum(np_pairwise_sum16(e, k), 1e-30f);
    w = e / d;
  } else if (mode == 2 || mode == 4) {
    // route_experts: exp(v - m) (norm_topk=1, m the largest selected value)
    // or exp(v) (norm_topk=0) over a float64 running sum, weights 0 when
    // the sum is not > 0 (blocks/moe.py:104-118).  The reference's m is a
    // float64 starting at -1e30, above the float32 slot filler -1e30f: a row
    // with nothing selected has exp(v - m) = 0 in every slot, so weights 0.
    const float m = mode == 4 ? wave_max(mine ? my_v : -1.0e30f) : 0.f;
    const float e = mine && (mode == 2 || m > -1.0e30f) ? expf(my_v - m) : 0.f;
    double s = 0.0;
    for (int j = 0; j < k; ++j) s += (double)lane_f(e, j);
    w = s > 0.0 ? (float)((double)e / s) : 0.f;
  }
  w_out = w;
  id_out = my_i;
}

}  // namespace ccq
