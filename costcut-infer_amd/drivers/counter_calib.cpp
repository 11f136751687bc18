// Calibration of the FETCH_SIZE / WRITE_SIZE counters: a streaming read of
// 64 MiB and a streaming write of 64 MiB (16-byte accesses, grid-stride),
// three dispatches each.  The counters' KiB per dispatch against 65536 KiB
// give the factors that turn a kernel's counters into HBM bytes.
// Build: hipcc -O2 --offload-arch=gfx950 costcut-infer_amd/drivers/counter_calib.cpp -o <binary>
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
__global__ __launch_bounds__(256) void calib_read(const u32x4* __restrict__ p, int64_t n16, uint32_t* out) {
  uint32_t acc = 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
    const u32x4 v = p[i];
    acc ^= v[0] + v[1] + v[2] + v[3];
  }
  if (acc == 0x12345678u) out[blockIdx.x] = acc;
}
__global__ __launch_bounds__(256) void calib_write(u32x4* __restrict__ p, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
    p[i] = u32x4{(uint32_t)i, 1u, 2u, 3u};
}
int main() {
  const int64_t R = 64ll << 20;
  void *a, *b, *o;
  if (hipMalloc(&a, R) || hipMalloc(&b, R) || hipMalloc(&o, 1 << 20)) return 3;
  if (hipMemset(a, 1, R) || hipDeviceSynchronize()) return 3;
  for (int r = 0; r < 3; ++r) {
    hipLaunchKernelGGL(calib_read, dim3(2048), dim3(256), 0, 0, (const u32x4*)a, R / 16, (uint32_t*)o);
    hipLaunchKernelGGL(calib_write, dim3(2048), dim3(256), 0, 0, (u32x4*)b, R / 16);
  }
  if (hipDeviceSynchronize()) return 4;
  printf("calib: read %lld B, write %lld B per dispatch, 3 each\n", (long long)R, (long long)R);
  return 0;
}
