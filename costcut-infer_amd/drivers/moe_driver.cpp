// Torch-free driver of the MoE entry points, for rocprofv3 runs (counter
// collection does not mix with the PyTorch runtime): synthetic weights
// (random packed words) and routing built on the host.
//   moe_driver w4  T reps   int4 prefill: 128 experts top-8 (skewed router),
//                           hidden 2048, inter 768, ccq_moe_w4_ffn
//   moe_driver w4d T reps   int4 decode: 64 experts top-6, hidden 2048,
//                           inter 1408, ccq_moe_w4_ffn on host-routed ids
//   moe_driver w4f T reps   the same layer from router logits,
//                           ccq_moe_w4_forward (prints the distinct experts)
//   moe_driver fp8 T reps   FP8 block prefill: 256 experts top-8, hidden
//                           7168, inter 2048, ccq_moe_fp8_ffn
//   moe_driver gemm M K N reps copies
//                           AWQ g128 linear y [M, N] = x [M, K] @ W,
//                           ccq_w4_gemm over `copies` rotating weight sets
//   moe_driver f8r T reps   MoE layer on per-row FP8 experts (the reference
//                           checkpoint's format): 256 experts top-8, hidden
//                           2048, inter 512, float32 activations,
//                           ccq_moe_fp8row_ffn (prints the distinct experts)
//   moe_driver f32 M K N reps
//                           float32 y [M, N] = x [M, K] @ w^T, w [N, K]
//                           (the router), ccq_f32_gemm with its workspace
//   moe_driver wq fmt M K N reps copies
//                           decoded-weight MFMA linear (float32 x and y),
//                           ccq_wq_mfma_linear_f32: fmt 0 FP8 row scale,
//                           1 INT8 row scale, 2 MXFP8, 3 MXFP4 (E8M0 scales
//                           per 32 columns)
// Build: hipcc -O2 -Iinclude costcut-infer_amd/drivers/moe_driver.cpp
//        -Lcostcut-infer_amd/ccut/_lib -lccq_hip -Wl,-rpath,<that dir> -o <binary>
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <cmath>
#include <vector>
#include <random>
#include <algorithm>
#include "ccq.h"
#define CK(x) do { hipError_t e = (x); if (e) { printf("hip error %d at %d\n", (int)e, __LINE__); exit(3); } } while (0)
static void* dalloc(size_t n) { void* p; CK(hipMalloc(&p, n < 256 ? 256 : n)); return p; }
static void fill_rand_u32(void* d, size_t words, uint32_t seed, uint32_t mask, uint32_t orv) {
  std::vector<uint32_t> h(words);
  std::mt19937 g(seed);
  for (auto& v : h) v = (g() & mask) | orv;
  CK(hipMemcpy(d, h.data(), words * 4, hipMemcpyHostToDevice));
}
static int run_gemm(int argc, char** argv) {
  const int64_t M = argc > 2 ? atoll(argv[2]) : 1, K = argc > 3 ? atoll(argv[3]) : 2048,
                N = argc > 4 ? atoll(argv[4]) : 5632;
  const int reps = argc > 5 ? atoi(argv[5]) : 20, copies = argc > 6 ? atoi(argv[6]) : 16;
  const int64_t szw = ccq_awq_sz_words(K, 128);
  std::vector<void*> w(copies), z(copies);
  for (int c = 0; c < copies; ++c) {
    w[c] = dalloc(K * N / 2);
    fill_rand_u32(w[c], K * N / 8, 11 + c, ~0u, 0);
    z[c] = dalloc(N * szw * 4);
    fill_rand_u32(z[c], N * szw, 101 + c, 0x000F007Fu, 0x3C00u);
  }
  void* x = dalloc(M * K * 2);
  fill_rand_u32(x, M * K / 2, 7, 0x807F807Fu, 0x3F003F00u);
  void* y = dalloc(M * N * 2);
  const size_t wsb = ccq_w4_gemm_workspace_size(M, K, N, 128);
  void* ws = wsb ? dalloc(wsb) : nullptr;
  for (int r = 0; r < reps; ++r) {
    const int c = r % copies;
    const int rc = ccq_w4_gemm(x, CCQ_F16, (const int32_t*)w[c], (const uint32_t*)z[c], CCQ_F16, y, CCQ_F16, M, K, N,
                               128, ws, wsb, nullptr);
    if (rc) { printf("rc=%d %s\n", rc, ccq_last_error()); return 4; }
  }
  CK(hipDeviceSynchronize());
  printf("gemm M=%lld K=%lld N=%lld reps %d copies %d done\n", (long long)M, (long long)K, (long long)N, reps, copies);
  return 0;
}

static int run_wq(int argc, char** argv) {
  const int fmt = argc > 2 ? atoi(argv[2]) : 3;
  const int64_t M = argc > 3 ? atoll(argv[3]) : 16, K = argc > 4 ? atoll(argv[4]) : 4096,
                N = argc > 5 ? atoll(argv[5]) : 14336;
  const int reps = argc > 6 ? atoi(argv[6]) : 24, copies = argc > 7 ? atoi(argv[7]) : 12;
  const int64_t wbytes = fmt == 3 ? N * K / 2 : N * K;
  const bool mx = fmt >= 2;
  std::vector<void*> w(copies);
  for (int c = 0; c < copies; ++c) {
    w[c] = dalloc(wbytes);
    fill_rand_u32(w[c], wbytes / 4, 11 + c, 0x77777777u, 0);  // finite e4m3 / int8 / 4-bit codes
  }
  void* sc = mx ? dalloc(N * K / 32) : dalloc(N * 4);
  if (mx)
    fill_rand_u32(sc, N * K / 128, 5, 0x03030303u, 0x7C7C7C7Cu);  // E8M0 124..127
  else
    fill_rand_u32(sc, N, 5, 0x007FFFFFu, 0x3C000000u);  // float scales in [2^-7, 2^-6)
  void* x = dalloc(M * K * 4);
  fill_rand_u32(x, M * K, 7, 0x807FFFFFu, 0x3F000000u);  // floats of magnitude [0.5, 1)
  void* y = dalloc(M * N * 4);
  for (int r = 0; r < reps; ++r) {
    const int c = r % copies;
    const int rc = ccq_wq_mfma_linear_f32((const float*)x, (const uint8_t*)w[c], sc, (float*)y, M, K, N, fmt, 32,
                                          1.0f, nullptr);
    if (rc) { printf("rc=%d %s\n", rc, ccq_last_error()); return 4; }
  }
  CK(hipDeviceSynchronize());
  printf("wq fmt=%d M=%lld K=%lld N=%lld reps %d copies %d done\n", fmt, (long long)M, (long long)K, (long long)N, reps,
         copies);
  return 0;
}

static int run_f8r(int argc, char** argv) {
  const int64_t T = argc > 2 ? atoll(argv[2]) : 16;
  const int reps = argc > 3 ? atoi(argv[3]) : 12;
  const int64_t E = 256, H = 2048, I = 512, k = 8;
  std::mt19937 g(91);
  std::vector<int64_t> ids(T * k);
  std::vector<float> wts(T * k, 1.0f / k);
  std::vector<int> used(E, 0);
  for (int64_t t = 0; t < T; ++t) {  // k distinct experts per token
    std::vector<int> perm(E);
    for (int e = 0; e < E; ++e) perm[e] = e;
    std::shuffle(perm.begin(), perm.end(), g);
    for (int j = 0; j < k; ++j) { ids[t * k + j] = perm[j]; used[perm[j]] = 1; }
  }
  int u = 0;
  for (int x : used) u += x;
  printf("f8r T=%lld: %d distinct experts routed\n", (long long)T, u);
  int64_t* d_ids = (int64_t*)dalloc(T * k * 8);
  float* d_w = (float*)dalloc(T * k * 4);
  CK(hipMemcpy(d_ids, ids.data(), T * k * 8, hipMemcpyHostToDevice));
  CK(hipMemcpy(d_w, wts.data(), T * k * 4, hipMemcpyHostToDevice));
  ccq_fp8row_experts ex = {};
  void* wg = dalloc(E * I * H); fill_rand_u32(wg, E * I * H / 4, 1, 0xB7B7B7B7u, 0x20202020u);  // finite e4m3
  void* wu = dalloc(E * I * H); fill_rand_u32(wu, E * I * H / 4, 2, 0xB7B7B7B7u, 0x20202020u);
  void* wd = dalloc(E * H * I); fill_rand_u32(wd, E * H * I / 4, 3, 0xB7B7B7B7u, 0x20202020u);
  void* sg = dalloc(E * I * 4); fill_rand_u32(sg, E * I, 4, 0x007FFFFFu, 0x3C000000u);
  void* su = dalloc(E * I * 4); fill_rand_u32(su, E * I, 5, 0x007FFFFFu, 0x3C000000u);
  void* sd = dalloc(E * H * 4); fill_rand_u32(sd, E * H, 6, 0x007FFFFFu, 0x3C000000u);
  ex.w_gate = (const uint8_t*)wg; ex.s_gate = (const float*)sg;
  ex.w_up = (const uint8_t*)wu; ex.s_up = (const float*)su;
  ex.w_down = (const uint8_t*)wd; ex.s_down = (const float*)sd;
  ex.num_experts = E; ex.hidden = H; ex.inter = I;
  void* x = dalloc(T * H * 4);
  fill_rand_u32(x, T * H, 7, 0x807FFFFFu, 0x3F000000u);  // floats of magnitude [0.5, 1)
  void* y = dalloc(T * H * 4);
  const size_t wsb = ccq_moe_fp8row_workspace_size(T, k, &ex);
  void* ws = dalloc(wsb);
  for (int r = 0; r < reps; ++r) {
    const int rc = ccq_moe_fp8row_ffn((const float*)x, d_ids, d_w, y, CCQ_F32, T, k, &ex, ws, wsb, nullptr);
    if (rc) { printf("rc=%d %s\n", rc, ccq_last_error()); return 4; }
  }
  CK(hipDeviceSynchronize());
  printf("f8r T=%lld workspace %zu bytes, reps %d done\n", (long long)T, wsb, reps);
  return 0;
}

static int run_f32(int argc, char** argv) {
  const int64_t M = argc > 2 ? atoll(argv[2]) : 16, K = argc > 3 ? atoll(argv[3]) : 2048,
                N = argc > 4 ? atoll(argv[4]) : 64;
  const int reps = argc > 5 ? atoi(argv[5]) : 20;
  void* x = dalloc(M * K * 4); fill_rand_u32(x, M * K, 7, 0x807FFFFFu, 0x3F000000u);
  void* w = dalloc(N * K * 4); fill_rand_u32(w, N * K, 8, 0x807FFFFFu, 0x3C000000u);
  void* y = dalloc(M * N * 4);
  const size_t wsb = ccq_f32_gemm_workspace_size(M, K, N);
  void* ws = wsb ? dalloc(wsb) : nullptr;
  for (int r = 0; r < reps; ++r) {
    const int rc = ccq_f32_gemm((const float*)x, (const float*)w, (float*)y, M, K, N, 1, ws, wsb, nullptr);
    if (rc) { printf("rc=%d %s\n", rc, ccq_last_error()); return 4; }
  }
  CK(hipDeviceSynchronize());
  printf("f32 M=%lld K=%lld N=%lld workspace %zu reps %d done\n", (long long)M, (long long)K, (long long)N, wsb, reps);
  return 0;
}

int main(int argc, char** argv) {
  if (argc > 1 && !strcmp(argv[1], "f8r")) return run_f8r(argc, argv);
  if (argc > 1 && !strcmp(argv[1], "f32")) return run_f32(argc, argv);
  if (argc > 1 && !strcmp(argv[1], "gemm")) return run_gemm(argc, argv);
  if (argc > 1 && !strcmp(argv[1], "wq")) return run_wq(argc, argv);
  const bool fp8 = argc > 1 && !strcmp(argv[1], "fp8");
  const bool fwd = argc > 1 && !strcmp(argv[1], "w4f");  // decode shape through ccq_moe_w4_forward (logits)
  const bool dec = fwd || (argc > 1 && !strcmp(argv[1], "w4d"));  // int4 MoE decode shape
  const int64_t T = argc > 2 ? atoll(argv[2]) : 4096;
  const int reps = argc > 3 ? atoi(argv[3]) : 5;
  const int64_t E = fp8 ? 256 : (dec ? 64 : 128), H = fp8 ? 7168 : 2048, I = fp8 ? 2048 : (dec ? 1408 : 768),
                k = dec ? 6 : 8;
  const double skew = fp8 || dec ? 0.0 : 2.0;
  // routing: logits N(0,1) + per-expert bias N(0, skew), top-k, softmax over the k
  std::mt19937 g(75);
  std::normal_distribution<float> nd(0.f, 1.f);
  std::vector<float> bias(E);
  for (auto& b : bias) b = (float)(nd(g) * skew);
  std::vector<int64_t> ids(T * k);
  std::vector<float> wts(T * k);
  std::vector<std::pair<float, int>> v(E);
  for (int64_t t = 0; t < T; ++t) {
    for (int e = 0; e < E; ++e) v[e] = {nd(g) + bias[e], e};
    std::partial_sort(v.begin(), v.begin() + k, v.end(), [](auto a, auto b) { return a.first > b.first; });
    float m = v[0].first, s = 0.f;
    for (int j = 0; j < k; ++j) s += expf(v[j].first - m);
    for (int j = 0; j < k; ++j) { ids[t * k + j] = v[j].second; wts[t * k + j] = expf(v[j].first - m) / s; }
  }
  std::vector<float> lg(T * E);
  for (auto& l : lg) l = nd(g);
  if (fwd) {  // distinct experts of the logits' top-k (for the algorithmic bytes)
    std::vector<int> used(E, 0);
    for (int64_t t = 0; t < T; ++t) {
      for (int e = 0; e < E; ++e) v[e] = {lg[t * E + e], e};
      std::partial_sort(v.begin(), v.begin() + k, v.end(), [](auto a, auto b) { return a.first > b.first; });
      for (int j = 0; j < k; ++j) used[v[j].second] = 1;
    }
    int u = 0;
    for (int x : used) u += x;
    printf("w4f T=%lld: %d distinct experts routed\n", (long long)T, u);
  }
  float* d_lg = (float*)dalloc(T * E * 4);
  CK(hipMemcpy(d_lg, lg.data(), T * E * 4, hipMemcpyHostToDevice));
  int64_t* d_ids = (int64_t*)dalloc(T * k * 8);
  float* d_w = (float*)dalloc(T * k * 4);
  CK(hipMemcpy(d_ids, ids.data(), T * k * 8, hipMemcpyHostToDevice));
  CK(hipMemcpy(d_w, wts.data(), T * k * 4, hipMemcpyHostToDevice));
  // activations bf16 ~ small values (random mantissa, exponent around 1)
  void* x = dalloc(T * H * 2);
  fill_rand_u32(x, T * H / 2, 7, 0x807F807Fu, 0x3F003F00u);
  void* y = dalloc(T * H * 2);
  int rc;
  size_t wsb;
  if (!fp8) {
    const int64_t szw = ccq_awq_sz_words(H, 128), szw2 = ccq_awq_sz_words(I, 128);
    ccq_w4_experts ex = {};
    void* wg = dalloc(E * H * I / 2); fill_rand_u32(wg, E * H * I / 8, 1, ~0u, 0);
    void* wu = dalloc(E * H * I / 2); fill_rand_u32(wu, E * H * I / 8, 2, ~0u, 0);
    void* wd = dalloc(E * H * I / 2); fill_rand_u32(wd, E * H * I / 8, 3, ~0u, 0);
    // scale bits: bf16 ~0.01 (0x3C23), zero 0..15
    void* zg = dalloc(E * I * szw * 4); fill_rand_u32(zg, E * I * szw, 4, 0x000F007Fu, 0x3C000000u >> 16);
    void* zu = dalloc(E * I * szw * 4); fill_rand_u32(zu, E * I * szw, 5, 0x000F007Fu, 0x3C00u);
    void* zd = dalloc(E * H * szw2 * 4); fill_rand_u32(zd, E * H * szw2, 6, 0x000F007Fu, 0x3C00u);
    ex.w_gate = (const int32_t*)wg; ex.sz_gate = (const uint32_t*)zg;
    ex.w_up = (const int32_t*)wu; ex.sz_up = (const uint32_t*)zu;
    ex.w_down = (const int32_t*)wd; ex.sz_down = (const uint32_t*)zd;
    ex.scale_dtype = CCQ_BF16; ex.num_experts = E; ex.hidden = H; ex.inter = I; ex.group_size = 128;
    wsb = ccq_moe_w4_workspace_size(T, k, &ex);
    void* ws = dalloc(wsb);
    for (int r = 0; r < reps; ++r) {
      rc = fwd ? ccq_moe_w4_forward(x, CCQ_BF16, d_lg, T, k, 1, nullptr, nullptr, y, CCQ_BF16, &ex, ws, wsb, nullptr)
               : ccq_moe_w4_ffn(x, CCQ_BF16, d_ids, d_w, y, CCQ_BF16, T, k, &ex, ws, wsb, nullptr);
      if (rc) { printf("rc=%d %s\n", rc, ccq_last_error()); return 4; }
    }
  } else {
    ccq_fp8_experts ex = {};
    void* wg = dalloc(E * H * I); fill_rand_u32(wg, E * H * I / 4, 1, 0xB7B7B7B7u, 0x20202020u);
    void* wu = dalloc(E * H * I); fill_rand_u32(wu, E * H * I / 4, 2, 0xB7B7B7B7u, 0x20202020u);
    void* wd = dalloc(E * H * I); fill_rand_u32(wd, E * H * I / 4, 3, 0xB7B7B7B7u, 0x20202020u);
    const int64_t sgu = E * (I / 128) * (H / 128), sd = E * (H / 128) * (I / 128);
    void* s1 = dalloc(sgu * 4); fill_rand_u32(s1, sgu, 4, 0x007FFFFFu, 0x3C000000u);
    void* s2 = dalloc(sgu * 4); fill_rand_u32(s2, sgu, 5, 0x007FFFFFu, 0x3C000000u);
    void* s3 = dalloc(sd * 4); fill_rand_u32(s3, sd, 6, 0x007FFFFFu, 0x3C000000u);
    ex.w_gate = (const uint8_t*)wg; ex.s_gate = (const float*)s1;
    ex.w_up = (const uint8_t*)wu; ex.s_up = (const float*)s2;
    ex.w_down = (const uint8_t*)wd; ex.s_down = (const float*)s3;
    ex.num_experts = E; ex.hidden = H; ex.inter = I;
    wsb = ccq_moe_fp8_workspace_size(T, k, &ex);
    void* ws = dalloc(wsb);
    for (int r = 0; r < reps; ++r) {
      rc = ccq_moe_fp8_ffn(x, CCQ_BF16, d_ids, d_w, y, CCQ_BF16, T, k, &ex, ws, wsb, nullptr);
      if (rc) { printf("rc=%d %s\n", rc, ccq_last_error()); return 4; }
    }
  }
  CK(hipDeviceSynchronize());
  printf("%s T=%lld workspace %zu bytes, reps %d done\n", argc > 1 ? argv[1] : "w4", (long long)T, wsb, reps);
  return 0;
}
